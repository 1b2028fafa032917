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


def keep_blocks(keep) -> torch.Tensor:
    """A boolean keep mask [M, K] (numpy or torch; K % 8 == 0) in the kernels' 8 x 8 block bit
    layout: uint8 [ceil(M / 8), K], row group R = rows 8 R .. 8 R + 7, byte 8 b + i = row
    8 R + i's bits of columns 8 b .. 8 b + 7 (bit j = column 8 b + j); rows past M zero."""
    import numpy as np

    keep = np.asarray(keep.numpy() if isinstance(keep, torch.Tensor) else keep, dtype=bool)
    M, K = keep.shape
    Mp = (M + 7) // 8 * 8
    padded = np.zeros((Mp, K), dtype=bool)
    padded[:M] = keep
    rows = np.packbits(padded, axis=1, bitorder="little")  # [Mp, K / 8], one byte per row
    return torch.from_numpy(
        np.ascontiguousarray(rows.reshape(Mp // 8, 8, K // 8).transpose(0, 2, 1).reshape(Mp // 8, K)))


def keep_rows(bits: torch.Tensor, M: int):
    """The inverse of keep_blocks on rows < M: numpy uint8 [M, K / 8], byte c / 8 of row m holding
    columns c .. c + 7 (np.packbits(keep, axis=1, bitorder="little") of the mask)."""
    b = bits.cpu().numpy()
    G, K = b.shape
    rows = b.reshape(G, K // 8, 8).transpose(0, 2, 1).reshape(G * 8, K // 8)
    return rows[:M]
