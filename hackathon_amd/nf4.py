"""NF4 dequantisation and the 4-bit linear layers that use it (drop-in for solution/nf4.py).

Every 4-bit layer call rebuilds the weight from the packed NF4 nibbles and the
double-quantised block scales (solution/nf4.py:1-16); here that rebuild is the gfx950 kernel
`qlora_nf4_dequant`, with the scale dequantisation `code2[q] * absmax2 + offset` folded in and
evaluated with the same fp32 operation order, so the weights come out bit-identical to the
reference's formula. A bf16/fp16 contraction runs in the library's MFMA GEMM (`qlora_gemm`);
an fp32 one (bitsandbytes' default compute dtype) runs in torch's fp32 GEMM on the kernel's
fp32 weight, as the reference does. The backward re-dequantises (nothing dense is kept
between forward and backward, solution/nf4.py:95-112).

Signatures kept from the reference: `dequantize_nf4(packed, quant_state, dtype)`,
`supported(qs)`, `NF4Linear.apply(x, packed, quant_state, bias)`, `_prepare(module, x)`,
`linear4bit(module, x, keep_compute_dtype)`, `patch_linear4bit()`, `project(layer, x)`.
"""

from __future__ import annotations

import torch

from . import _lib
from . import gemm as _gemm
from . import quant

DEQUANT_BLOCK = 1024  # packed bytes per workgroup step in the reference (solution/nf4.py:22)

_NF4_TABLES = {}


def _nf4_table(device):
    """The 16-entry fp32 NF4 codebook on `device`, cached per device (solution/nf4.py:52-62)."""
    table = _NF4_TABLES.get(device)
    if table is None:
        table = quant.nf4_code(device).contiguous()
        _NF4_TABLES[device] = table
    return table


def supported(quant_state):
    """NF4, 2-D, even blocksizes (solution/nf4.py:65-68)."""
    return (quant_state is not None and quant_state.quant_type == "nf4"
            and len(quant_state.shape) == 2 and quant_state.blocksize % 2 == 0
            and (not quant_state.nested or quant_state.state2.blocksize % 2 == 0))


def _offset_value(quant_state):
    """The double-quant offset as a Python float. Reading it from a device tensor
    synchronises the host (solution/nf4.py:81 does so on every call, 392 times per 7B step)
    and is not allowed under graph capture, so the value is read once per offset tensor and
    cached on the state; assigning a new offset tensor, or changing it in place (which bumps
    its version counter), invalidates the cache."""
    off = quant_state.offset
    version = getattr(off, "_version", None)
    cached = getattr(quant_state, "_ql_offset", None)
    if cached is not None and cached[0] is off and cached[1] == version:
        return cached[2]
    value = float(off)
    try:
        quant_state._ql_offset = (off, version, value)
    except AttributeError:  # a state object that takes no new attributes
        pass
    return value


def _scale_args(quant_state):
    """(absmax, nested, code2, absmax2, offset, blocksize2) for the C-ABI (solution/nf4.py:77-86)."""
    if quant_state.nested:
        s2 = quant_state.state2
        absmax = quant_state.absmax
        if absmax.dtype != torch.uint8:
            raise TypeError("double-quantised absmax must be uint8 codes")
        code2 = s2.code if s2.code.dtype == torch.float32 else s2.code.float()
        absmax2 = s2.absmax if s2.absmax.dtype == torch.float32 else s2.absmax.float()
        if code2.numel() != 256:
            raise ValueError("the double-quant code map must have 256 entries")
        return (absmax.contiguous(), 1, code2.contiguous(), absmax2.contiguous(),
                _offset_value(quant_state), int(s2.blocksize))
    absmax = quant_state.absmax
    absmax = (absmax if absmax.dtype == torch.float32 else absmax.float()).contiguous()
    return absmax, 0, None, None, 0.0, 1


def dequantize_nf4(packed, quant_state, dtype=torch.float16, out=None):
    """The weight [out_features, in_features] in `dtype`, from the packed NF4 bytes
    (solution/nf4.py:71-92)."""
    shape = tuple(quant_state.shape)
    _lib.require_device(packed)
    if out is None:
        out = torch.empty(shape, dtype=dtype, device=packed.device)
    n = out.numel()
    packed = packed.reshape(-1)
    if packed.numel() * 2 < n:
        raise ValueError("packed buffer is smaller than the quantised shape")
    absmax, nested, code2, absmax2, offset, blocksize2 = _scale_args(quant_state)
    _lib.call("qlora_nf4_dequant", packed.data_ptr(), n, absmax.data_ptr(), nested,
              _lib.ptr(code2), _lib.ptr(absmax2), offset, int(quant_state.blocksize),
              blocksize2, _nf4_table(packed.device).data_ptr(), out.data_ptr(),
              _lib.tag(out.dtype), _lib.stream_of(out))
    return out


def dequantize_nf4_t(packed, quant_state, dtype=torch.bfloat16, out=None):
    """The TRANSPOSED weight [in_features, out_features] in `dtype` (bit-identical to
    dequantize_nf4(...).t()), for the k-contiguous backward GEMM dY @ W."""
    rows, cols = tuple(quant_state.shape)
    _lib.require_device(packed)
    if out is None:
        out = torch.empty((cols, rows), dtype=dtype, device=packed.device)
    absmax, nested, code2, absmax2, offset, blocksize2 = _scale_args(quant_state)
    _lib.call("qlora_nf4_dequant_t", packed.reshape(-1).data_ptr(), rows, cols, absmax.data_ptr(),
              nested, _lib.ptr(code2), _lib.ptr(absmax2), offset, int(quant_state.blocksize),
              blocksize2, _nf4_table(packed.device).data_ptr(), out.data_ptr(), out.stride(0),
              _lib.tag(out.dtype), _lib.stream_of(out))
    return out


def _pow2_at_least(v, lo):
    v = int(v)
    return v >= lo and v & (v - 1) == 0


def _groupable(items, outs, transposed):
    """Whether qlora_nf4_dequant_group / _t_group take these weights and outputs."""
    if not 2 <= len(items) <= 4 or len({bool(qs.nested) for _, qs in items}) != 1:
        return False
    lds = set()
    for (packed, qs), out in zip(items, outs):
        rows, cols = (int(v) for v in qs.shape)
        align = 16 if transposed else 4
        if (not packed.is_cuda or not packed.is_contiguous() or packed.device != out.device
                or packed.data_ptr() % align
                or out.data_ptr() % 16 or not _pow2_at_least(qs.blocksize, 16 if transposed else 8)
                or (qs.nested and not _pow2_at_least(qs.state2.blocksize, 1))
                or packed.numel() * 2 < rows * cols):
            return False
        if transposed:
            if (cols % 128 or rows % 8 or out.dtype not in (torch.bfloat16, torch.float16)
                    or tuple(out.shape) != (cols, rows) or out.stride(1) != 1):
                return False
            lds.add(out.stride(0))
        elif (rows * cols) % 8 or out.numel() != rows * cols or not out.is_contiguous():
            return False
    return not transposed or (len(lds) == 1 and lds.pop() % 8 == 0)


def _group_call(name, items, outs, dtype, *extra):
    keep = []  # the scale tensors _scale_args made stay alive until the launch is queued
    arr = (_lib.Nf4Weight * len(items))()
    for i, ((packed, qs), out) in enumerate(zip(items, outs)):
        absmax, nested, code2, absmax2, offset, blocksize2 = _scale_args(qs)
        keep += [absmax, code2, absmax2]
        rows, cols = (int(v) for v in qs.shape)
        arr[i] = _lib.Nf4Weight(packed.data_ptr(), rows, cols, absmax.data_ptr(), _lib.ptr(code2),
                                _lib.ptr(absmax2), offset, int(qs.blocksize), blocksize2,
                                out.data_ptr())
    device = outs[0].device
    _lib.call(name, arr, len(items), int(bool(items[0][1].nested)), _nf4_table(device).data_ptr(),
              *extra, _lib.tag(dtype), _lib.stream_of(outs[0]))


def dequantize_nf4_group(items, dtype, outs):
    """Dequantise the weights `items` = [(packed, quant_state), ...] into `outs` (one
    contiguous [out_features, in_features] tensor of `dtype` each): one launch for up to four
    weights of the same nesting (qlora_nf4_dequant_group), else one dequantize_nf4 each.
    Bit-identical either way."""
    for out in outs:
        _lib.require_device(out)
    if _groupable(items, outs, False) and all(o.dtype == dtype for o in outs):
        _group_call("qlora_nf4_dequant_group", items, outs, dtype)
    else:
        for (packed, qs), out in zip(items, outs):
            dequantize_nf4(packed, qs, dtype, out=out)
    return outs


def dequantize_nf4_t_group(items, dtype, outs):
    """The transposed weights of `items` into `outs` ([in_features, out_features] column blocks
    of one buffer, sharing its row stride): one launch (qlora_nf4_dequant_t_group) when the
    weights qualify, else one dequantize_nf4_t each. Bit-identical either way."""
    for out in outs:
        _lib.require_device(out)
    if _groupable(items, outs, True) and all(o.dtype == dtype for o in outs):
        _group_call("qlora_nf4_dequant_t_group", items, outs, dtype, outs[0].stride(0))
    else:
        for (packed, qs), out in zip(items, outs):
            dequantize_nf4_t(packed, qs, dtype, out=out)
    return outs


# Token rows up to which the forward GEMM dequantises W inside the GEMM (gemm_nf4) instead of
# writing a dense 16-bit W first. Measured on MI355X at the Qwen2.5-7B projection shapes: the
# fused GEMM is 1.12-1.28x faster at 64 and 256 rows (W's dense write and re-read dominate),
# 0.83-0.98x at 512 and 0.63-0.72x at 4096 (every 256-row tile of x redoes the dequantisation).
FUSED_GEMM_MAX_ROWS = 256


def use_fused_gemm(x2, quant_state, packed, a2=None):
    """Whether the forward of x2 [M, K] (with the rank-16 segment a2 when given) against this
    NF4 weight takes gemm_nf4."""
    return x2.shape[0] <= FUSED_GEMM_MAX_ROWS and fused_gemm_ok(quant_state, packed, x2, a2)


GEMM_NF4_MAX_K2 = 64  # the second K segment is one K step of the tile (qlora_gemm_nf4)


def fused_gemm_ok(quant_state, packed, x=None, a2=None):
    """Whether gemm_nf4 takes this weight (and input x [M, K], segment a2 [M, K2] when given):
    in_features a multiple of 64, blocksize a power of two >= 64 dividing it (blocksize2 a
    power of two), packed codes 16-B aligned; x 16-bit, 16-B aligned rows of unit stride;
    K2 a multiple of 64 and at most 64."""
    if packed.data_ptr() % 16:
        return False
    if a2 is not None and (a2.shape[1] % 64 or a2.shape[1] > GEMM_NF4_MAX_K2):
        return False
    _, cols = tuple(quant_state.shape)
    bs = int(quant_state.blocksize)
    if cols % 64 or bs < 64 or bs & (bs - 1) or cols % bs:
        return False
    if quant_state.nested:
        bs2 = int(quant_state.state2.blocksize)
        if bs2 < 1 or bs2 & (bs2 - 1):
            return False
    if x is not None:
        if x.dtype not in (torch.bfloat16, torch.float16) or x.stride(-1) != 1:
            return False
        if x.data_ptr() % 16 or x.stride(0) % 8:
            return False
    return True


def gemm_nf4(x, packed, quant_state, out=None, a2=None, b2=None, bias=None, alpha=1.0):
    """out = alpha * (x @ W^T + a2 @ b2^T) (+ bias) with W [N, K] the NF4 weight of
    `quant_state`, dequantised inside the GEMM to x's dtype (bit-identical to the GEMM on
    dequantize_nf4(packed, quant_state, x.dtype)); a2 [M, K2] and b2 [N, K2] are the optional
    rank-16 segment (K2 = 64: one K step) (qlora_gemm_nf4). x [M, K] 2-D."""
    _lib.require_device(x, packed)
    N, K = tuple(quant_state.shape)
    M = x.shape[0]
    if x.shape[1] != K:
        raise ValueError(f"x has {x.shape[1]} columns, the weight {K}")
    if out is None:
        out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    K2 = 0 if a2 is None else a2.shape[1]
    absmax, nested, code2, absmax2, offset, blocksize2 = _scale_args(quant_state)
    ws, ws_bytes = _lib.workspace("qlora_gemm_nf4_workspace_size", M, N, K, device=x.device)
    bias = bias.to(x.dtype).contiguous() if bias is not None else None
    _lib.call("qlora_gemm_nf4", M, N, K, x.data_ptr(), x.stride(0), packed.reshape(-1).data_ptr(),
              absmax.data_ptr(), nested, _lib.ptr(code2), _lib.ptr(absmax2), offset,
              int(quant_state.blocksize), blocksize2, _nf4_table(packed.device).data_ptr(), K2,
              _lib.ptr(a2), a2.stride(0) if a2 is not None else 0, _lib.ptr(b2),
              b2.stride(0) if b2 is not None else 0, _lib.tag(x.dtype), out.data_ptr(),
              out.stride(0), _lib.ptr(bias), float(alpha), _lib.ptr(ws), ws_bytes,
              _lib.stream_of(x))
    return out


def transposed_dequant_ok(quant_state, packed=None):
    """Whether dequantize_nf4_t takes this weight: in_features % 128 == 0,
    out_features % 8 == 0, blocksize a power of two >= 16 (and, when given, the packed codes
    16-B aligned)."""
    if packed is not None and packed.data_ptr() % 16:
        return False
    rows, cols = tuple(quant_state.shape)
    bs = int(quant_state.blocksize)
    ok = cols % 128 == 0 and rows % 8 == 0 and bs >= 16 and bs & (bs - 1) == 0
    if ok and quant_state.nested:
        bs2 = int(quant_state.state2.blocksize)
        ok = bs2 > 0 and bs2 & (bs2 - 1) == 0
    return ok


class NF4Linear(torch.autograd.Function):
    """y = x @ W.T + b with W rebuilt by the dequant kernel in forward and again in backward
    (solution/nf4.py:95-112). Weight and bias are frozen."""

    @staticmethod
    def forward(ctx, x, packed, quant_state, bias):
        x2 = x.reshape(-1, x.shape[-1])
        ctx.packed, ctx.quant_state = packed, quant_state
        if x2.dtype in (torch.bfloat16, torch.float16) and use_fused_gemm(x2, quant_state, packed):
            out = gemm_nf4(x2, packed, quant_state, bias=bias)  # W dequantised in the GEMM
            return out.view(*x.shape[:-1], out.shape[-1])
        weight = dequantize_nf4(packed, quant_state, x.dtype)
        if x.dtype == torch.float32:
            # fp32 compute (bitsandbytes' default compute dtype): the library's MFMA GEMMs take
            # 16-bit operands, so the fp32 product is torch's, on the kernel's fp32 W, as in
            # solution/nf4.py:100-102
            return torch.nn.functional.linear(x, weight, bias)
        return _gemm.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, grad_out):
        grad_x = None
        if ctx.needs_input_grad[0]:
            qs = ctx.quant_state
            rows = tuple(qs.shape)[0]
            if grad_out.dtype == torch.float32:
                weight = dequantize_nf4(ctx.packed, qs, torch.float32)
                grad_x = torch.matmul(grad_out, weight)                # solution/nf4.py:110-111
            elif grad_out.dtype in (torch.bfloat16, torch.float16) \
                    and transposed_dequant_ok(qs, ctx.packed) and rows % 64 == 0:
                # dY @ W as an NT GEMM against W^T, dequantised straight into that layout
                weight_t = dequantize_nf4_t(ctx.packed, qs, grad_out.dtype)
                grad_x = _gemm.linear(grad_out, weight_t)
            else:
                weight = dequantize_nf4(ctx.packed, qs, grad_out.dtype)
                grad_x = _gemm.matmul_nn(grad_out, weight)
        return grad_x, None, None, None


def _prepare(module, x):
    """The part of a 4-bit layer's forward before the matmul (solution/nf4.py:115-138):
    returns (x, bias, input dtype), or None when this layer should take the original path.
    bf16 compute is accepted here (the reference accepted fp16/fp32 only, :131-132); fp32
    compute runs NF4Linear's fp32 branch (the kernel's fp32 W and torch's fp32 GEMM)."""
    quant_state = getattr(module.weight, "quant_state", None)
    if (not x.is_cuda or not supported(quant_state) or module.weight.requires_grad
            or (module.bias is not None and module.bias.requires_grad)):
        return None
    if not module.compute_type_is_set:
        module.set_compute_type(x)
        module.compute_type_is_set = True
    inp_dtype = x.dtype
    if module.compute_dtype is not None:
        x = x.to(module.compute_dtype)
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return None
    bias = module.bias
    if bias is not None:
        if bias.dtype != x.dtype:
            bias.data = bias.data.to(x.dtype)
        bias = bias.to(x.dtype)
    return x, bias, inp_dtype


def _original_forward(module, x):
    """The unpatched 4-bit forward: torch-op dequantisation + F.linear in the compute dtype
    (what bitsandbytes' Linear4bit.forward computes). Used for inputs the kernels do not take
    (CPU or meta tensors) and as the eager baseline."""
    from . import eager

    return eager.linear4bit_eager(module, x)


_ORIGINAL = {}


def linear4bit(module, x, keep_compute_dtype=False):
    """A 4-bit layer's forward with the dequant kernel (solution/nf4.py:141-149). With
    keep_compute_dtype the output stays in the compute dtype instead of the input dtype."""
    prepared = _prepare(module, x)
    if prepared is None:
        return _ORIGINAL.get("forward", _original_forward)(module, x)
    x, bias, inp_dtype = prepared
    out = NF4Linear.apply(x, module.weight, module.weight.quant_state, bias)
    return out if keep_compute_dtype else out.to(inp_dtype)


def patch_linear4bit():
    """Route bitsandbytes' Linear4bit.forward through `linear4bit` when bitsandbytes is
    importable (solution/nf4.py:155-166); this package's own Linear4bit always does."""
    try:
        import bitsandbytes.nn.modules as bnb_modules
    except ImportError:
        return
    cls = bnb_modules.Linear4bit
    if "forward" in _ORIGINAL:
        return
    _ORIGINAL["forward"] = cls.forward

    def forward(self, x):
        return linear4bit(self, x)

    cls.forward = forward


def project(layer, x):
    """An MLP projection that keeps its output in the compute dtype when it is a plain 4-bit
    layer (solution/nf4.py:169-175). Anything else runs as it is."""
    if type(layer) is quant.Linear4bit:
        return linear4bit(layer, x, keep_compute_dtype=True)
    return layer(x)
