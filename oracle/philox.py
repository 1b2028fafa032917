"""Dropout-mask oracle: Philox4x32-10 and the uniform Triton's tl.rand draws (numpy).

The reference's mask is `keep = tl.rand(seed, (row*N + col).to(int32)) > p`
(solution/lora.py:41-43). tl.rand (triton/language/random.py, installed Triton 3.6) runs
Philox4x32 for 10 rounds on counter {offset as uint32, 0, 0, 0} and key {seed lo, seed hi},
takes word 0 as int32, folds negatives to -x-1, and multiplies by 4.6566127342e-10 in fp32.
Philox is the published generator of Salmon et al., "Parallel Random Numbers: As Easy as
1, 2, 3" (SC'11). Test infrastructure only.

Pins (tests/test_oracle_ops.py): the Random123 known-answer vectors for philox4x32-10, and
vectors drawn from Triton's own tl.rand under its CPU interpreter (tests/golden/).
"""

from __future__ import annotations

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
SCALE = np.float32(4.6566127342e-10)


def philox4x32_10(c0, c1, c2, c3, k0, k1):
    """Vectorised Philox4x32-10. All inputs uint32 arrays (broadcastable); returns 4 words."""
    c0, c1, c2, c3 = (np.asarray(c, dtype=np.uint32) for c in (c0, c1, c2, c3))
    k0, k1 = np.asarray(k0, dtype=np.uint32), np.asarray(k1, dtype=np.uint32)
    for _ in range(10):
        p0 = c0.astype(np.uint64) * M0
        p1 = c2.astype(np.uint64) * M1
        hi0, lo0 = (p0 >> np.uint64(32)).astype(np.uint32), p0.astype(np.uint32)
        hi1, lo1 = (p1 >> np.uint64(32)).astype(np.uint32), p1.astype(np.uint32)
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
        k0 = ((k0.astype(np.uint64) + np.uint64(W0)) & np.uint64(0xFFFFFFFF)).astype(np.uint32)
        k1 = ((k1.astype(np.uint64) + np.uint64(W1)) & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    return c0, c1, c2, c3


def uniform(seed: int, offsets) -> np.ndarray:
    """tl.rand(seed, int32 offsets) as float32."""
    offs = np.asarray(offsets, dtype=np.int64).astype(np.int32).view(np.uint32)
    seed = int(seed) & 0xFFFF_FFFF_FFFF_FFFF
    z = np.zeros_like(offs)
    w0, _, _, _ = philox4x32_10(offs, z, z, z, np.uint32(seed & 0xFFFFFFFF), np.uint32(seed >> 32))
    x = w0.view(np.int32)
    x = np.where(x < 0, ~x, x)  # -x - 1
    return (x.astype(np.float32) * SCALE).astype(np.float32)


def keep_mask(seed: int, n_rows: int, n_cols: int, p: float) -> np.ndarray:
    """The reference's dropout keep mask for an [n_rows, n_cols] input."""
    flat = (np.arange(n_rows, dtype=np.int64)[:, None] * n_cols
            + np.arange(n_cols, dtype=np.int64)[None, :])
    return uniform(seed, flat.astype(np.int32)) > np.float32(p)
