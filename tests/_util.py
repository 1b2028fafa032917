"""Test constants mirroring solution/_testing.py:8-12, plus small helpers."""

import torch

DEVICE = "cuda"
TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
# bf16 tolerances the kernel set is held to (rtol = atol = 1e-2 for RMSNorm/RoPE/SwiGLU)
BF16_TOL = dict(rtol=1e-2, atol=1e-2)


def bits16(t: torch.Tensor) -> torch.Tensor:
    """Raw 16-bit patterns of a bf16/fp16 tensor (for bit-exact comparison)."""
    return t.contiguous().view(torch.int16)


def seeded(seed: int = 0) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g
