"""Small helpers shared by the patches (solution/_common.py:6-25)."""

import torch


def on_gpu(*tensors):
    """True when every argument is a tensor on a GPU device (torch on ROCm reports HIP devices
    as `is_cuda`). Every patch checks this first and otherwise keeps the original code path
    (solution/_common.py:6-9)."""
    return all(isinstance(t, torch.Tensor) and t.is_cuda for t in tensors)


def autocast_dtype():
    """The dtype a matmul runs in right now: the autocast dtype if autocast is on, else None
    (solution/_common.py:12-16)."""
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return None


def round_mode(dtype):
    """0: keep fp32, 1: round through fp16, 2: round through bf16 (solution/_common.py:19-25)."""
    if dtype == torch.float16:
        return 1
    if dtype == torch.bfloat16:
        return 2
    return 0
