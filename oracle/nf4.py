"""NF4 dequant oracle: the C restatement (nf4_oracle.c) through ctypes, plus a numpy twin.

Reference: solution/nf4.py:25-49 (kernel) and :71-92 (QuantState unpacking). Test
infrastructure only.

Pins (tests/test_oracle_nf4.py): the published NF4 codebook fixture and its scipy
re-derivation; hand-computed known-answer bytes (nibble order, block index, scale order);
a crafted case where a fused multiply-add would round differently; nibble 7 -> 0 and
nibble 0/15 -> -s/+s; quantise -> dequantise -> quantise idempotence; bf16 rounding against
torch's conversion.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "_build" / "liboracle.so"
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            from . import build

            build.build()
        L = ctypes.CDLL(str(_LIB_PATH))
        P, I64, I, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        for name in ("oracle_nf4_dequant_f32", "oracle_nf4_dequant_bf16"):
            fn = getattr(L, name)
            fn.argtypes = [P, I64, P, I, P, P, F, I64, I64, P, P]
            fn.restype = None
        L.oracle_nf4_scales.argtypes = [I64, P, I, P, P, F, I64, P]
        L.oracle_nf4_scales.restype = None
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _np(a, dtype):
    return np.ascontiguousarray(np.asarray(a, dtype=dtype))


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def unpack_state(state):
    """numpy views of a QuantState-like object's fields (any device)."""
    def cpu(t):
        return t.detach().cpu().numpy() if hasattr(t, "detach") else np.asarray(t)
    nested = bool(state.nested)
    if nested:
        s2 = state.state2
        return dict(absmax=_np(cpu(state.absmax), np.uint8), nested=1,
                    code2=_np(cpu(s2.code), np.float32), absmax2=_np(cpu(s2.absmax), np.float32),
                    offset=np.float32(float(state.offset)), blocksize=int(state.blocksize),
                    blocksize2=int(s2.blocksize))
    return dict(absmax=_np(cpu(state.absmax), np.float32), nested=0, code2=None, absmax2=None,
                offset=np.float32(0.0), blocksize=int(state.blocksize), blocksize2=1)


def dequant(packed, n_weights, table, *, absmax, nested, code2, absmax2, offset, blocksize,
            blocksize2, out="bf16"):
    """C oracle. Returns uint16 bf16 bits (out='bf16') or float32 (out='f32')."""
    packed = _np(packed, np.uint8).reshape(-1)
    table = _np(table, np.float32)
    if packed.size * 2 < n_weights:
        raise ValueError("packed too small")
    res = np.empty(n_weights, np.uint16 if out == "bf16" else np.float32)
    fn = lib().oracle_nf4_dequant_bf16 if out == "bf16" else lib().oracle_nf4_dequant_f32
    fn(_p(packed), n_weights, _p(absmax), nested, _p(code2), _p(absmax2), float(offset),
       blocksize, blocksize2, _p(table), _p(res))
    return res


def dequant_state(packed, state, table, out="bf16"):
    n = int(np.prod(tuple(state.shape)))
    return dequant(packed.detach().cpu().numpy() if hasattr(packed, "detach") else packed, n,
                   table, out=out, **unpack_state(state))


def scales(n_blocks, *, absmax, nested, code2, absmax2, offset, blocksize2, **_):
    res = np.empty(n_blocks, np.float32)
    lib().oracle_nf4_scales(n_blocks, _p(absmax), nested, _p(code2), _p(absmax2), float(offset),
                            blocksize2, _p(res))
    return res


def f32_to_bf16_bits(x) -> np.ndarray:
    x = _np(x, np.float32).reshape(-1)
    f = lib().oracle_f32_to_bf16
    return np.array([f(float(v)) for v in x], dtype=np.uint16)


def dequant_numpy(packed, n_weights, table, *, absmax, nested, code2, absmax2, offset,
                  blocksize, blocksize2):
    """numpy twin of the C oracle's fp32 result (same operation order, float32 throughout)."""
    p = _np(packed, np.uint8).reshape(-1)
    j = np.arange(n_weights)
    nib = np.where(j & 1, p[j >> 1] & 15, p[j >> 1] >> 4).astype(np.int64)
    b = j // blocksize
    if nested:
        s = (np.float32(1) * code2[absmax[b]] * absmax2[b // blocksize2]).astype(np.float32)
        s = (s + np.float32(offset)).astype(np.float32)
    else:
        s = absmax[b].astype(np.float32)
    return (table[nib].astype(np.float32) * s).astype(np.float32)


def dequant_torch(packed, state, table, out_dtype=None):
    """Torch restatement on the CPU, vectorised over every weight (runs on all of torch's
    intra-op threads): the reference's dequant (solution/nf4.py:26-49) with the same fp32
    operation order as the C oracle: s = code2[q] * absmax2[b // bs2], s = s + offset,
    w = nf4[c] * s, each rounded to fp32, then one RNE conversion to `out_dtype` (bf16 by
    default). Used as the CPU baseline of the dequant; pinned bit-exact to the C oracle."""
    import torch

    st = unpack_state(state)
    p = torch.as_tensor(packed).reshape(-1).to(torch.uint8)
    n = int(np.prod(tuple(state.shape)))
    nib = torch.stack(((p >> 4) & 15, p & 15), dim=1).reshape(-1)[:n].long()
    bs = st["blocksize"]
    nb = -(-n // bs)
    if st["nested"]:
        q = torch.from_numpy(st["absmax"]).long()
        code2 = torch.from_numpy(st["code2"])
        a2 = torch.from_numpy(st["absmax2"])
        s = code2[q] * a2[torch.arange(nb) // st["blocksize2"]]
        s = s + torch.tensor(st["offset"], dtype=torch.float32)
    else:
        s = torch.from_numpy(st["absmax"]).float()
    tab = torch.as_tensor(np.asarray(table, np.float32))
    w = tab[nib]
    full = (n // bs) * bs
    head = (w[:full].view(-1, bs) * s[: n // bs, None]).reshape(-1)
    if full < n:
        head = torch.cat([head, w[full:] * s[-1]])
    return head.to(out_dtype or torch.bfloat16)
