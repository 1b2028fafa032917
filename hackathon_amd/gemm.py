"""Host wrappers of the library's MFMA GEMM (`qlora_gemm`).

These stand in for the torch GEMM calls of the reference's path (F.linear and torch.matmul
in solution/nf4.py:102,111, the LoRA nn.Linear pair of solution/lora.py:172 and the chunk
GEMMs of solution/cross_entropy.py:117,123 / solution/fused_ce.py:135,143). Inputs must be
bf16 or fp16 on a GPU; they are made unit-stride along their contiguous dimension if needed.
"""

from __future__ import annotations

import ctypes

import weakref

import torch

from . import _lib


def _rows(t: torch.Tensor) -> torch.Tensor:
    """A 2-D view with unit stride along the last dim (any row stride: the kernel takes it)."""
    t2 = t.reshape(-1, t.shape[-1])
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) < t2.shape[1]):
        t2 = t2.contiguous()
    return t2


def padded_rows(n_rows: int, n_cols: int, dtype, device) -> torch.Tensor:
    """An [n_rows, n_cols] buffer whose rows start 16-B aligned (row stride rounded up to a
    multiple of 8 elements), so the GEMM and row kernels take their vector paths."""
    stride = (n_cols + 7) // 8 * 8
    return torch.empty((n_rows, stride), dtype=dtype, device=device)[:, :n_cols]


_NN_VIA_T_MIN_M = 512  # below this many rows the transpose would cost more than it saves


def gemm(a: torch.Tensor, b: torch.Tensor, *, a_km: bool = False, b_kn: bool = False,
         out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
         bias: torch.Tensor | None = None, alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """C = alpha * A @ B^T (+ beta C) (+ bias) with A [M,K] (or stored [K,M] when a_km) and
    B [N,K] (or stored [K,N] when b_kn), both 2-D, unit stride along their last dim.
    Split-K workspace, when the library asks for one, comes from torch's caching allocator.
    A large NN product (b_kn, M >= 512, K % 64 == 0) transposes B into a temporary and takes
    the NT kernel."""
    _lib.require_device(a, b)
    if a.dtype != b.dtype or a.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"GEMM operands must share dtype bf16/fp16, got {a.dtype}, {b.dtype}")
    a, b = _rows(a), _rows(b)
    M, K = (a.shape[1], a.shape[0]) if a_km else (a.shape[0], a.shape[1])
    N, Kb = (b.shape[1], b.shape[0]) if b_kn else (b.shape[0], b.shape[1])
    if K != Kb:
        raise ValueError(f"GEMM inner sizes differ: {K} vs {Kb}")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype or a.dtype, device=a.device)
    elif out.shape != (M, N) or out.stride(-1) != 1:
        raise ValueError("out must be [M, N] with unit stride along N")
    if bias is not None:
        bias = bias.to(a.dtype).contiguous()
    if b_kn and not a_km and M >= _NN_VIA_T_MIN_M and N >= 64 and K % 64 == 0:
        # B stored [K, N]: one tiled transpose (2·K·N·2 bytes of traffic) puts it k-contiguous,
        # and the large-tile NT kernel then runs at about twice the general kernel's rate
        b, b_kn = transpose16(b), False
    ws_bytes = int(_lib.load().qlora_gemm_workspace_size(int(a_km), int(b_kn), M, N, K))
    ws = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=out.device) \
        if ws_bytes > 0 else None
    _lib.call("qlora_gemm_ws", int(a_km), int(b_kn), M, N, K, a.data_ptr(), a.stride(0),
              b.data_ptr(), b.stride(0), _lib.tag(a.dtype), out.data_ptr(), out.stride(0),
              _lib.tag(out.dtype), _lib.ptr(bias), float(alpha), float(beta), _lib.ptr(ws),
              ws_bytes, _lib.stream_of(out))
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """F.linear(x, weight, bias) for x [..., K] and weight [N, K] (output in x.dtype)."""
    x2 = _rows(x)
    y = gemm(x2, weight, bias=bias)
    return y.view(*x.shape[:-1], weight.shape[0])


def matmul_nn(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a @ b for a [..., K] and b [K, N] (output in a.dtype)."""
    a2 = _rows(a)
    y = gemm(a2, b, b_kn=True)
    return y.view(*a.shape[:-1], b.shape[1])


def matmul_tn(a: torch.Tensor, b: torch.Tensor, out_dtype=None) -> torch.Tensor:
    """a^T @ b for a [K, M] and b [K, N], both stored row-major (reduction over rows)."""
    return gemm(_rows(a), _rows(b), a_km=True, b_kn=True, out_dtype=out_dtype)


def transpose16(t: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """t.T as a contiguous [cols, rows] tensor (16-bit dtypes), by the library's tiled
    transpose; `out` may be a wider buffer view whose rows are `rows` long."""
    _lib.require_device(t)
    if t.element_size() != 2 or t.dim() != 2:
        raise TypeError("transpose16 takes a 2-D 16-bit tensor")
    t2 = t if t.stride(-1) == 1 else t.contiguous()
    rows, cols = t2.shape
    if out is None:
        out = torch.empty((cols, rows), dtype=t.dtype, device=t.device)
    _lib.call("qlora_transpose16", t2.data_ptr(), rows, cols, t2.stride(0), out.data_ptr(),
              out.stride(0), _lib.stream_of(t2))
    return out


_FROZEN: dict = {}


def _frozen(w: torch.Tensor, kind, make):
    """make(w), kept while `w` is alive and unmodified (same storage, same version) under the
    key (w, kind): operands derived once from frozen weights that every step reads."""
    key = (id(w), kind)
    hit = _FROZEN.get(key)
    if hit is not None:
        ref, ptr, version, derived = hit
        if ref() is w and ptr == w.data_ptr() and version == w._version:
            return derived
    for k in [k for k, v in _FROZEN.items() if v[0]() is None]:
        del _FROZEN[k]
    derived = make(w)
    _FROZEN[key] = (weakref.ref(w), w.data_ptr(), w._version, derived)
    return derived


def transposed_frozen(w: torch.Tensor) -> torch.Tensor:
    """w.T, contiguous, kept while `w` is alive and unmodified. For frozen weights read every
    step in the other orientation (the lm_head in dz @ W): the transpose is paid once, not per
    call."""
    return _frozen(w, "T", transpose16)


def frozen_as(w: torch.Tensor, dtype) -> torch.Tensor:
    """w in `dtype`, contiguous: `w` itself when it already is, else a copy kept while `w` is
    alive, unmodified and frozen (a weight that requires grad is cast on every call)."""
    if w.dtype == dtype and w.is_contiguous():
        return w
    if w.requires_grad:
        return w.detach().to(dtype).contiguous()
    return _frozen(w, dtype, lambda t: t.to(dtype).contiguous())


def gemm_nt_cat(a: torch.Tensor, b: torch.Tensor, a2: torch.Tensor | None,
                b2: torch.Tensor | None, out: torch.Tensor, bias: torch.Tensor | None = None,
                alpha: float = 1.0, residual: torch.Tensor | None = None) -> torch.Tensor:
    """out = alpha * (a @ b^T + a2 @ b2^T) (+ bias) in one NT GEMM over the concatenated K
    (qlora_gemm_nt_cat). All operands 2-D, unit stride along K, K and K2 multiples of 64.
    With `residual` ([M, N], out's 16-bit dtype; no bias, alpha 1) out = residual + the
    product, each rounded as `residual + (a @ b^T + a2 @ b2^T)` rounds them
    (qlora_gemm_nt_cat_residual)."""
    M, K = a.shape
    N = b.shape[0]
    K2 = 0 if a2 is None else a2.shape[1]
    ws, ws_bytes = _lib.workspace("qlora_gemm_nt_cat_workspace_size", M, N, K, device=out.device)
    if residual is not None:
        if bias is not None or alpha != 1.0 or residual.dtype != out.dtype:
            raise ValueError("a residual takes no bias, alpha 1 and out's dtype")
        if residual.shape != (M, N) or residual.stride(-1) != 1:
            raise ValueError(f"residual must be [{M}, {N}] with unit column stride")
        _lib.call("qlora_gemm_nt_cat_residual", M, N, K, a.data_ptr(), a.stride(0), b.data_ptr(),
                  b.stride(0), K2, _lib.ptr(a2), a2.stride(0) if a2 is not None else 0,
                  _lib.ptr(b2), b2.stride(0) if b2 is not None else 0, _lib.tag(a.dtype),
                  out.data_ptr(), out.stride(0), _lib.tag(out.dtype), residual.data_ptr(),
                  residual.stride(0), _lib.ptr(ws), ws_bytes, _lib.stream_of(out))
        return out
    _lib.call("qlora_gemm_nt_cat", M, N, K, a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0),
              K2, _lib.ptr(a2), a2.stride(0) if a2 is not None else 0, _lib.ptr(b2),
              b2.stride(0) if b2 is not None else 0, _lib.tag(a.dtype), out.data_ptr(),
              out.stride(0), _lib.tag(out.dtype), _lib.ptr(bias), float(alpha), _lib.ptr(ws),
              ws_bytes, _lib.stream_of(out))
    return out


def _slots(rows: int, what: str) -> int:
    if rows % 16 or not 16 <= rows <= 64:
        raise ValueError(f"{what} must have 16, 32, 48 or 64 rows (1-4 rank-16 adapters), got {rows}")
    return rows // 16


def lora_down(x: torch.Tensor, y: torch.Tensor, out: torch.Tensor, alpha: float = 1.0,
              out_t: torch.Tensor | None = None) -> torch.Tensor:
    """out[:, :16G] = alpha * x @ y^T (y [16G, K]: G <= 4 rank-16 adapters that read x) and
    out[:, 16G:] = 0 (qlora_lora_down, x read once); with `out_t` ([16G, >= M], x's dtype)
    also the 16G columns transposed, the operand lora_wgrad takes."""
    _lib.require_rows(x.dtype, x=x, y=y, out_t=out_t)
    _lib.require_rows(out.dtype, out=out)
    M, K = x.shape
    slots = _slots(y.shape[0], "y")
    ws, ws_bytes = _lib.workspace("qlora_lora_down_workspace_size", M, K, slots, device=x.device)
    _lib.call("qlora_lora_down", x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0), M, K,
              slots, _lib.tag(x.dtype), out.data_ptr(), out.stride(0), out.shape[1],
              _lib.tag(out.dtype), float(alpha), _lib.ptr(out_t),
              out_t.stride(0) if out_t is not None else 0, _lib.ptr(ws), ws_bytes,
              _lib.stream_of(x))
    return out


def lora_t_buffer(m: int, dtype, device, rows: int = 16) -> torch.Tensor:
    """A [rows, m] buffer for lora_down's transposed output (row stride a multiple of 8)."""
    return torch.empty((rows, (m + 7) // 8 * 8), dtype=dtype, device=device)[:, :m]


def lora_wgrad_diag(pt: torch.Tensor, q: torch.Tensor, col_offsets, alphas) -> torch.Tensor:
    """The lora_B gradients of G adapters with concatenated outputs from one pass: fp32 [N, 16]
    whose rows off_i .. off_{i+1} - 1 are alphas[i] * q[:, off_i:off_{i+1}]^T pt[16 i:16 i + 16]^T
    (pt = the adapters' stacked u^T [16 G, M], q = their concatenated output gradient [M, N])
    (qlora_lora_wgrad_diag)."""
    _lib.require_rows(q.dtype, pt=pt, q=q)
    M, N = q.shape
    G = _slots(pt.shape[0], "pt")
    if len(col_offsets) != G + 1 or len(alphas) != G:
        raise ValueError("col_offsets needs G + 1 entries and alphas G")
    out = torch.empty((N, 16), dtype=torch.float32, device=q.device)
    ws, ws_bytes = _lib.workspace("qlora_lora_wgrad_diag_workspace_size", M, N, G,
                                  device=q.device)
    offs = _lib.i64_array(col_offsets)
    al = (ctypes.c_float * G)(*[float(a) for a in alphas])
    _lib.call("qlora_lora_wgrad_diag", pt.data_ptr(), pt.stride(0), q.data_ptr(), q.stride(0), M,
              N, G, _lib.tag(q.dtype), offs, al, out.data_ptr(), _lib.ptr(ws), ws_bytes,
              _lib.stream_of(q))
    return out


def lora_wgrad(pt: torch.Tensor, q: torch.Tensor, alpha: float = 1.0,
               transposed: bool = False) -> torch.Tensor:
    """fp32 alpha * q^T @ pt^T for q [M, N] and pt [16G, M] (token-contiguous, as lora_down's
    `out_t`; G <= 4 adapters whose gradients reduce over the same q, q read once)
    (qlora_lora_wgrad): [N, 16G], or [16G, N] when `transposed`."""
    _lib.require_rows(q.dtype, q=q, pt=pt)
    M, N = q.shape
    slots = _slots(pt.shape[0], "pt")
    nc = 16 * slots
    out = torch.empty((nc, N) if transposed else (N, nc), dtype=torch.float32, device=q.device)
    ws, ws_bytes = _lib.workspace("qlora_lora_wgrad_workspace_size", M, N, slots,
                                  device=q.device)
    _lib.call("qlora_lora_wgrad", pt.data_ptr(), pt.stride(0), q.data_ptr(), q.stride(0), M, N,
              slots, _lib.tag(q.dtype), out.data_ptr(), int(transposed), float(alpha),
              _lib.ptr(ws), ws_bytes, _lib.stream_of(q))
    return out


def lora_wgrad_masked(pt: torch.Tensor, q: torch.Tensor, bitss, p: float,
                      alpha: float = 1.0) -> torch.Tensor:
    """fp32 [16 G, N]: rows 16 g .. 16 g + 15 = alpha * pt_g q_g, q_g = adapter g's dropout of
    q [M, N] (keep bits bitss[g] from lora.dropout_with_bits / dropout_down, scale 1 / (1 - p)),
    for G <= 4 adapters in one pass over q (qlora_lora_wgrad_masked): the lora_A gradients of a
    group's adapters without their dropped inputs stored."""
    import ctypes

    _lib.require_rows(q.dtype, q=q, pt=pt)
    M, N = q.shape
    slots = _slots(pt.shape[0], "pt")
    if len(bitss) != slots or len({b.stride(0) for b in bitss}) != 1:
        raise ValueError("one keep-bit tensor per adapter, all with one group stride")
    out = torch.empty((16 * slots, N), dtype=torch.float32, device=q.device)
    ws, ws_bytes = _lib.workspace("qlora_lora_wgrad_workspace_size", M, N, slots,
                                  device=q.device)
    ptrs = (ctypes.c_void_p * slots)(*[b.data_ptr() for b in bitss])
    _lib.call("qlora_lora_wgrad_masked", pt.data_ptr(), pt.stride(0), q.data_ptr(), q.stride(0),
              M, N, slots, _lib.tag(q.dtype), ptrs, bitss[0].stride(0), 1.0 / (1.0 - p),
              out.data_ptr(), float(alpha), _lib.ptr(ws), ws_bytes, _lib.stream_of(q))
    return out


def lora_pack(a: torch.Tensor, b: torch.Tensor, scaling: float, dtype, pad: int = 64):
    """(a16 [16,K], at_pad [K,pad], bs_pad [N,pad], bt [16,N]) in `dtype` from the fp32 adapter
    factors a [16, K] and b [N, 16] in one launch (qlora_lora_pack)."""
    _lib.require_device(a, b)
    a = a.detach().float().contiguous()
    b = b.detach().float().contiguous()
    K, N = a.shape[1], b.shape[0]
    dev = a.device
    a16 = torch.empty((16, K), dtype=dtype, device=dev)
    at = torch.empty((K, pad), dtype=dtype, device=dev)
    bs = torch.empty((N, pad), dtype=dtype, device=dev)
    bt = torch.empty((16, N), dtype=dtype, device=dev)
    _lib.call("qlora_lora_pack", a.data_ptr(), b.data_ptr(), K, N, float(scaling), _lib.tag(dtype),
              a16.data_ptr(), at.data_ptr(), bs.data_ptr(), bt.data_ptr(), pad, _lib.stream_of(a))
    return a16, at, bs, bt


def lora_pack_group(factors, dtype, pad: int = 64):
    """(a16 [16G, K], at_pad [K, pad], bs_pad [N, pad], bt [16G, N]) in `dtype` for G <= 4
    adapters (a_g [16, K], b_g [n_g, 16], scaling_g) that read the same input, adapter g in
    columns 16g .. 16g+15 and output rows off_g .. off_g + n_g - 1, N = sum n_g; bt is
    block-diagonal (B_g^T in rows 16g .. 16g+15 of adapter g's columns, zeros elsewhere)
    (qlora_lora_pack_group, one launch)."""
    items = []
    for a, b, s in factors:
        _lib.require_device(a, b)
        items.append((a.detach().float().contiguous(), b.detach().float().contiguous(), s))
    K = items[0][0].shape[1]
    N = sum(b.shape[0] for _, b, _ in items)
    G = len(items)
    dev = items[0][0].device
    a16 = torch.empty((16 * G, K), dtype=dtype, device=dev)
    at = torch.empty((K, pad), dtype=dtype, device=dev)
    bs = torch.empty((N, pad), dtype=dtype, device=dev)
    bt = torch.empty((16 * G, N), dtype=dtype, device=dev)
    _lib.call("qlora_lora_pack_group", _lib.lora_factors(items), G, K, _lib.tag(dtype),
              a16.data_ptr(), at.data_ptr(), bs.data_ptr(), bt.data_ptr(), pad,
              _lib.stream_of(a16))
    return a16, at, bs, bt
