"""LoRA dropout + cast and scaled add around a 4-bit LoRA layer (drop-in for solution/lora.py).

A peft 4-bit LoRA layer's forward under autocast (solution/lora.py:5-7):
    result = base_layer(x)
    out    = lora_B(lora_A(dropout(x))) * scaling
    result = result + out
Here (solution/lora.py:8-17):
    xd  = DropoutCast(x)   one pass: counter-based mask (regenerated in backward, never stored),
                           1/(1-p) scale, cast to the compute dtype  -> qlora_lora_dropout_scale
    lo  = lora_B(lora_A(xd))                                        -> qlora_gemm (x2)
    out = ScaledAdd(result, lo, scaling) in fp32                    -> qlora_lora_scaled_add
With dropout off and rank 16 on an NF4 base (the QLoRA step), the layer instead runs as
`LoraNF4Linear`: the adapter term rides inside the base GEMM as one extra K step, and the
adapter gradients come from dedicated rank-16 reduction kernels.
peft is not installed in this environment, so `LoraLinear4bit` below carries the attribute
surface the patched forward reads (base_layer, lora_A/lora_B/lora_dropout ModuleDicts,
scaling, active_adapters, disable_adapters, merged) and always runs the patched forward.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _common, _lib, adapter_packs
from . import gemm as _gemm

TORCH_DROPOUT_RNG = False


def _rows(t):
    t2 = t.reshape(-1, t.shape[-1])
    return t2 if t2.stride(-1) == 1 else t2.contiguous()


def _block(n):
    """The reference's per-row column block (solution/lora.py:68-71); the HIP kernels move 8
    elements per thread per step and do not need it."""
    return 1024


def _dropout_scale(src, out_dtype, seed, p, scale):
    """OUT = SRC * keep * scale, cast (solution/lora.py:74-81)."""
    _lib.require_device(src)
    s2 = _rows(src)
    out = torch.empty(s2.shape, dtype=out_dtype, device=src.device)
    M, N = s2.shape
    _lib.call("qlora_lora_dropout_scale", s2.data_ptr(), _lib.tag(s2.dtype), s2.stride(0),
              out.data_ptr(), _lib.tag(out_dtype), out.stride(0), M, N,
              int(seed) & 0xFFFF_FFFF_FFFF_FFFF, float(p), float(scale), _lib.stream_of(s2))
    return out.view(src.shape)


class DropoutCast(torch.autograd.Function):
    """solution/lora.py:84-93: the backward regenerates the same mask from the same seed."""

    @staticmethod
    def forward(ctx, x, p, seed, out_dtype):
        scale = 1.0 / (1.0 - p) if p > 0 else 1.0
        ctx.p, ctx.seed, ctx.scale, ctx.x_dtype = p, seed, scale, x.dtype
        return _dropout_scale(x, out_dtype, seed, p, scale)

    @staticmethod
    def backward(ctx, g):
        return _dropout_scale(g, ctx.x_dtype, ctx.seed, ctx.p, ctx.scale), None, None, None


class ScaledAdd(torch.autograd.Function):
    """out = base + lo * scaling in fp32 (solution/lora.py:96-112)."""

    @staticmethod
    def forward(ctx, base, lo, scaling):
        _lib.require_device(base, lo)
        b2, l2 = _rows(base), _rows(lo)
        out_dtype = torch.promote_types(base.dtype, lo.dtype)
        out = torch.empty(b2.shape, dtype=out_dtype, device=base.device)
        M, N = b2.shape
        _lib.call("qlora_lora_scaled_add", b2.data_ptr(), _lib.tag(b2.dtype), b2.stride(0),
                  l2.data_ptr(), _lib.tag(l2.dtype), l2.stride(0), out.data_ptr(),
                  _lib.tag(out_dtype), out.stride(0), M, N, float(scaling), _lib.stream_of(b2))
        ctx.scaling, ctx.base_dtype, ctx.lo_dtype = scaling, base.dtype, lo.dtype
        return out.view(base.shape)

    @staticmethod
    def backward(ctx, g):
        d_base = g if g.dtype == ctx.base_dtype else g.to(ctx.base_dtype)
        d_lo = _dropout_scale(g, ctx.lo_dtype, 0, 0.0, ctx.scaling)  # g * scaling, cast
        return d_base, d_lo, None


class _Seeds:
    """Dropout seeds from a private generator seeded from the run's torch seed, so the run is
    reproducible and no other random stream is disturbed (solution/lora.py:115-124)."""
    gen = None

    @classmethod
    def next(cls):
        if cls.gen is None:
            cls.gen = torch.Generator().manual_seed(torch.initial_seed() & 0xFFFF_FFFF)
        return int(torch.randint(0, 2**31 - 1, (1,), generator=cls.gen))


class LoRALinearFn(torch.autograd.Function):
    """lo = (xd @ A^T) @ B^T on the MFMA GEMM, with the adapter weight gradients:
        u = xd A^T;  lo = u B^T;   dB = dlo^T u;  du = dlo B;  dA = du^T xd;  dxd = du A
    (the nn.Linear pair of solution/lora.py:172 and what autograd computes for it).
    The MFMA GEMM takes 16-bit operands; with an fp32 compute dtype the same six products run
    on torch's fp32 GEMM, which is what the reference's nn.Linear pair runs in any dtype."""

    @staticmethod
    def forward(ctx, xd, a_weight, b_weight):
        x2 = _rows(xd)
        a = a_weight.to(x2.dtype)
        b = b_weight.to(x2.dtype)
        if x2.dtype == torch.float32:
            u = x2 @ a.t()
            lo = u @ b.t()
        else:
            u = _gemm.gemm(x2, a)
            lo = _gemm.gemm(u, b)
        ctx.save_for_backward(x2, u, a, b)
        ctx.shape, ctx.wdtypes = xd.shape, (a_weight.dtype, b_weight.dtype)
        return lo.view(*xd.shape[:-1], b.shape[0])

    @staticmethod
    def backward(ctx, dlo):
        x2, u, a, b = ctx.saved_tensors
        d2 = _rows(dlo).to(x2.dtype)
        da = db = dx = None
        if x2.dtype == torch.float32:
            du = d2 @ b                                                 # [M, r]
            if ctx.needs_input_grad[2]:
                db = (d2.t() @ u).to(ctx.wdtypes[1])
            if ctx.needs_input_grad[1]:
                da = (du.t() @ x2).to(ctx.wdtypes[0])
            if ctx.needs_input_grad[0]:
                dx = (du @ a).view(ctx.shape)
            return dx, da, db
        du = _gemm.gemm(d2, b, b_kn=True)                               # [M, r]
        if ctx.needs_input_grad[2]:
            db = _gemm.matmul_tn(d2, u, out_dtype=torch.float32).to(ctx.wdtypes[1])
        if ctx.needs_input_grad[1]:
            da = _gemm.matmul_tn(du, x2, out_dtype=torch.float32).to(ctx.wdtypes[0])
        if ctx.needs_input_grad[0]:
            dx = _gemm.gemm(du, a, b_kn=True).view(ctx.shape)
        return dx, da, db


_PAD = 64  # rank-16 factors are zero-padded to one 64-wide K step of the NT GEMM


def keep_bits_buffer(M, K, device):
    """Keep bits of an [M, K] input in the kernels' 8 x 8 block layout: uint8 [ceil(M / 8), K],
    row group R holding rows 8 R .. 8 R + 7, byte 8 (c / 8) + row % 8 the bits of columns
    c .. c + 7 (bit j = column c + j)."""
    return torch.empty(((M + 7) // 8, K), dtype=torch.uint8, device=device)


def dropout_with_bits(x2, p, seed):
    """(x2 * keep / (1 - p), keep bits in keep_bits_buffer's layout) in x2's dtype, the mask of
    DropoutCast(x2, p, seed) (qlora_lora_dropout_scale_bits)."""
    M, K = x2.shape
    if x2.data_ptr() % 16 or x2.stride(0) % 8:
        x2 = x2.contiguous() if x2.stride(0) % 8 else x2.clone()
    xd = torch.empty((M, K), dtype=x2.dtype, device=x2.device)
    bits = keep_bits_buffer(M, K, x2.device)
    _lib.call("qlora_lora_dropout_scale_bits", x2.data_ptr(), x2.stride(0), xd.data_ptr(),
              xd.stride(0), bits.data_ptr(), bits.stride(0), M, K, _lib.tag(x2.dtype),
              int(seed) & 0xFFFF_FFFF_FFFF_FFFF, float(p), 1.0 / (1.0 - p), _lib.stream_of(x2))
    return xd, bits


def dropout_down(x2, a16, p, seeds, u, ut=None, keep_xd=False):
    """Each adapter's keep mask and down-projection in one pass over x2, for the G <= 4 adapters
    of a group (adapter g: rows 16 g .. 16 g + 15 of a16 [16 G, K], seed seeds[g]): returns
    ([xd_g] if keep_xd else None, [keep bits_g]) as dropout_with_bits(x2, p, seeds[g]) returns
    them, and writes u[:, 16 g:16 g + 16] = xd_g a16_g^T (zeros in u's columns 16 G ..) and,
    when given, ut [16 G, M] = its transpose (qlora_lora_dropout_down). K must be a multiple
    of 64."""
    M, K = x2.shape
    G = len(seeds)
    if x2.data_ptr() % 16 or x2.stride(0) % 8:
        x2 = x2.contiguous() if x2.stride(0) % 8 else x2.clone()
    xds = ([torch.empty((M, K), dtype=x2.dtype, device=x2.device) for _ in range(G)]
           if keep_xd else None)
    bitss = [keep_bits_buffer(M, K, x2.device) for _ in range(G)]
    seed_arr = (ctypes.c_uint64 * G)(*[int(s) & 0xFFFF_FFFF_FFFF_FFFF for s in seeds])
    xd_ptrs = (ctypes.c_void_p * G)(*[t.data_ptr() for t in xds]) if keep_xd else None
    bit_ptrs = (ctypes.c_void_p * G)(*[t.data_ptr() for t in bitss])
    ws, ws_bytes = _lib.workspace("qlora_lora_dropout_down_workspace_size", M, K, G,
                                  device=x2.device)
    _lib.call("qlora_lora_dropout_down", x2.data_ptr(), x2.stride(0), a16.data_ptr(),
              a16.stride(0), M, K, G, _lib.tag(x2.dtype), seed_arr, float(p), 1.0 / (1.0 - p),
              xd_ptrs, K, bit_ptrs, K, u.data_ptr(), u.stride(0), u.shape[1],
              None if ut is None else ut.data_ptr(), 0 if ut is None else ut.stride(0),
              _lib.ptr(ws), ws_bytes, _lib.stream_of(x2))
    return xds, bitss


def up_masked_add(dx, du, a16, bits, p):
    """dx += keep * (du a16) / (1 - p) in place: the input gradient of the adapter term of a
    dropped input (du [M, 16] and a16 [16, K] in dx's dtype, row strides >= 16 and >= K; bits
    from dropout_with_bits) (qlora_lora_up_masked_add)."""
    M, K = dx.shape
    _lib.call("qlora_lora_up_masked_add", dx.data_ptr(), dx.stride(0), du.data_ptr(),
              du.stride(0), a16.data_ptr(), a16.stride(0), bits.data_ptr(), bits.stride(0), M, K,
              _lib.tag(dx.dtype), 1.0 / (1.0 - p), _lib.stream_of(dx))


def up_masked_add_slots(dx, du, a16, bitss, p):
    """up_masked_add for the G <= 4 adapters of a group in one pass over dx: adapter g's du in
    columns 16 g .. 16 g + 15 of du, its A in rows 16 g .. of a16, its mask bitss[g] (one row
    stride for all) (qlora_lora_up_masked_add_slots)."""
    M, K = dx.shape
    G = len(bitss)
    if len({b.stride(0) for b in bitss}) != 1:
        raise ValueError("the masks' bits must share one row stride")
    ptrs = (ctypes.c_void_p * G)(*[b.data_ptr() for b in bitss])
    _lib.call("qlora_lora_up_masked_add_slots", dx.data_ptr(), dx.stride(0), du.data_ptr(),
              du.stride(0), a16.data_ptr(), a16.stride(0), ptrs, bitss[0].stride(0), G, M, K,
              _lib.tag(dx.dtype), 1.0 / (1.0 - p), _lib.stream_of(dx))


class LoraNF4Linear(torch.autograd.Function):
    """The whole 4-bit LoRA linear (rank 16) as one MFMA GEMM per direction:

        forward   u = xd A^T                      qlora_lora_down  -> [M, 64], cols >= 16 zero
                  y = [x | u] [W | s B]^T + bias   qlora_gemm_nt_cat (W dequantised first)
        backward  du = s g B                      qlora_lora_down  (Y = B^T)
                  dx = [g | du] [W^T | A^T]^T      qlora_gemm_nt_cat (W^T dequantised directly)
                  dB = s g^T u,  dA = du^T xd      qlora_lora_wgrad (reductions over tokens)

    with xd = x when p = 0. With dropout (p > 0, the reference's training regime) xd =
    x * keep / (1 - p) is never stored: one pass of qlora_lora_dropout_down draws the mask of
    DropoutCast with the same seed (kept as bits) and forms u from xd on the way; the dX GEMM
    runs on the base term alone and qlora_lora_up_masked_add adds keep * (du A) / (1 - p); dA
    comes from x and the bits (qlora_lora_wgrad_masked).

    The same sums as base_layer(x) + ScaledAdd(B(A(dropout(x)))) of solution/lora.py:157-173
    with the adapter term accumulated in fp32 inside the base GEMM instead of rounded to the
    compute dtype and added in a separate pass; u, du and s*B are the compute-dtype values the
    reference's autocast GEMMs see (s = alpha / r = 2 scales B exactly)."""

    @staticmethod
    def forward(ctx, x, a_weight, b_weight, packed, quant_state, bias, scaling, p, seed):
        from . import nf4

        x2 = x.reshape(-1, x.shape[-1]).contiguous()
        dt = x2.dtype
        M, K = x2.shape
        N = int(quant_state.shape[0])
        # A, A^T|0, s*B|0 and B^T in the compute dtype, one launch (kept for the backward)
        a16, at, bs, bt = adapter_packs.pack(a_weight, b_weight, scaling, dt, _PAD)
        u = torch.empty((M, _PAD), dtype=dt, device=x2.device)
        ut = _gemm.lora_t_buffer(M, dt, x2.device)                     # u^T, for dB
        bits = None
        if p > 0 and K % 64 == 0:  # the keep bits and u in one pass over x
            _, (bits,) = dropout_down(x2, a16, p, (seed,), u, ut)
        elif p > 0:
            xd, bits = dropout_with_bits(x2, p, seed)
            _gemm.lora_down(xd, a16, u, out_t=ut)
            del xd
        else:
            _gemm.lora_down(x2, a16, u, out_t=ut)
        y = torch.empty((M, N), dtype=dt, device=x2.device)
        b16 = None if bias is None else bias.to(dt)
        if nf4.use_fused_gemm(x2, quant_state, packed, a2=u):  # few rows: W dequantised in-GEMM
            nf4.gemm_nf4(x2, packed, quant_state, out=y, a2=u, b2=bs, bias=b16)
        else:
            w = nf4.dequantize_nf4(packed, quant_state, dt)
            _gemm.gemm_nt_cat(x2, w, u, bs, y, bias=b16)
            del w
        del u
        ctx.save_for_backward(x2, ut, at, bt, a16 if p > 0 else None, bits)
        ctx.packed, ctx.quant_state, ctx.scaling = packed, quant_state, float(scaling)
        ctx.p = float(p)
        ctx.shape, ctx.wdtypes = x.shape, (a_weight.dtype, b_weight.dtype)
        return y.view(*x.shape[:-1], N)

    @staticmethod
    def backward(ctx, g):
        from . import nf4

        x2, ut, at, bt, a16, bits = ctx.saved_tensors
        dt = x2.dtype
        M, K = x2.shape
        g2 = _rows(g)
        if g2.dtype != dt:
            g2 = g2.to(dt)
        g2 = g2.contiguous()
        s = ctx.scaling
        du = torch.empty((M, _PAD), dtype=dt, device=g2.device)
        dut = _gemm.lora_t_buffer(M, dt, g2.device)
        _gemm.lora_down(g2, bt, du, alpha=s, out_t=dut)                 # du = s g B
        dx = da = db = None
        if ctx.needs_input_grad[0]:
            wt = nf4.dequantize_nf4_t(ctx.packed, ctx.quant_state, dt)  # [K, N]
            dx = torch.empty((M, K), dtype=dt, device=g2.device)
            if bits is None:
                _gemm.gemm_nt_cat(g2, wt, du, at, dx)
            else:
                _gemm.gemm_nt_cat(g2, wt, None, None, dx)
                up_masked_add(dx, du, a16, bits, ctx.p)
            del wt
            dx = dx.view(ctx.shape)
        if ctx.needs_input_grad[1]:                                     # [16, K] = du^T xd
            da = (_gemm.lora_wgrad(dut, x2, transposed=True) if bits is None
                  else _gemm.lora_wgrad_masked(dut, x2, [bits], ctx.p))  # xd from x and bits
            if da.dtype != ctx.wdtypes[0]:
                da = da.to(ctx.wdtypes[0])
        if ctx.needs_input_grad[2]:
            db = _gemm.lora_wgrad(ut, g2, alpha=s)                     # [N, 16] = s g^T u
            if db.dtype != ctx.wdtypes[1]:
                db = db.to(ctx.wdtypes[1])
        return dx, da, db, None, None, None, None, None, None


def _fused_base(layer, adapter, x, compute_dtype, p):
    """(packed, quant_state, bias) when the layer can run as LoraNF4Linear, else None: rank
    16, a frozen NF4 base whose shapes the k-contiguous kernels take, dropout off or drawn
    from this package's Philox stream (not torch's RNG, TORCH_DROPOUT_RNG)."""
    from . import nf4

    if compute_dtype not in (torch.bfloat16, torch.float16):
        return None
    if p != 0 and (TORCH_DROPOUT_RNG or not 0 < p < 1):
        return None
    base = layer.base_layer
    weight = getattr(base, "weight", None)
    qs = getattr(weight, "quant_state", None)
    if qs is None or not nf4.supported(qs) or weight.requires_grad or not weight.is_cuda:
        return None
    bias = getattr(base, "bias", None)
    if bias is not None and bias.requires_grad:
        return None
    a_w, b_w = layer.lora_A[adapter].weight, layer.lora_B[adapter].weight
    out_f, in_f = (int(d) for d in qs.shape)
    if a_w.shape != (16, in_f) or b_w.shape != (out_f, 16):
        return None
    if in_f % 128 or out_f % 64 or not nf4.transposed_dequant_ok(qs, weight):
        return None
    if not (a_w.is_cuda and b_w.is_cuda):
        return None
    return weight, qs, bias


def _single_adapter(layer):
    """The one active plain-Linear adapter, or None (solution/lora.py:127-142)."""
    if layer.disable_adapters or layer.merged:
        return None
    active = [a for a in layer.active_adapters if a in layer.lora_A.keys()]
    if len(active) != 1:
        return None
    a = active[0]
    if a in getattr(layer, "lora_variant", {}):
        return None
    lora_a, lora_b = layer.lora_A[a], layer.lora_B[a]
    if not (type(lora_a) is torch.nn.Linear and type(lora_b) is torch.nn.Linear
            and lora_a.bias is None and lora_b.bias is None):
        return None
    if not isinstance(layer.lora_dropout[a], (torch.nn.Dropout, torch.nn.Identity)):
        return None
    return a


def lora_forward(self, x, *args, **kwargs):
    """The patched 4-bit LoRA forward (solution/lora.py:157-173), or None when this call must
    take the layer's original path."""
    compute_dtype = _common.autocast_dtype() or getattr(self, "compute_dtype", None)
    adapter = None
    if not args and not kwargs and compute_dtype is not None and _common.on_gpu(x) \
            and x.dtype in (torch.float32, torch.float16, torch.bfloat16):
        adapter = _single_adapter(self)
    if adapter is None:
        return None
    drop = self.lora_dropout[adapter]
    p = float(drop.p) if isinstance(drop, torch.nn.Dropout) and drop.training else 0.0
    fused = _fused_base(self, adapter, x, compute_dtype, p)
    if fused is not None:
        weight, qs, bias = fused
        xc = x if x.dtype == compute_dtype else x.to(compute_dtype)
        with torch.autocast("cuda", enabled=False):
            y = LoraNF4Linear.apply(xc, self.lora_A[adapter].weight, self.lora_B[adapter].weight,
                                    weight, qs, bias, self.scaling[adapter], p,
                                    _Seeds.next() if p > 0 else 0)
        out_dtype = torch.promote_types(x.dtype, compute_dtype)
        return y if y.dtype == out_dtype else y.to(out_dtype)
    result = self.base_layer(x)
    if TORCH_DROPOUT_RNG and p > 0:
        xd = DropoutCast.apply(drop(x), 0.0, 0, compute_dtype)
    elif p == 0 and x.dtype == compute_dtype:
        xd = x  # dropout off and no cast to do: the kernel would copy x unchanged
    else:
        xd = DropoutCast.apply(x, p, _Seeds.next() if p > 0 else 0, compute_dtype)
    with torch.autocast("cuda", enabled=False):
        lo = LoRALinearFn.apply(xd, self.lora_A[adapter].weight, self.lora_B[adapter].weight)
    return ScaledAdd.apply(result, lo, self.scaling[adapter])


class LoraLinear4bit(torch.nn.Module):
    """A 4-bit base layer with one LoRA adapter, with peft's LoRA-layer attribute surface.

    `compute_dtype` is the adapters' matmul dtype when autocast is off (under autocast the
    autocast dtype wins, as in solution/lora.py:158)."""

    def __init__(self, base_layer, r=16, lora_alpha=32, lora_dropout=0.0, adapter="default",
                 compute_dtype=None, init_b_std=0.0):
        super().__init__()
        self.base_layer = base_layer
        in_f, out_f = base_layer.in_features, base_layer.out_features
        dev = base_layer.bias.device if base_layer.bias is not None else (
            base_layer.weight.device if base_layer.weight is not None else None)
        self.lora_A = torch.nn.ModuleDict(
            {adapter: torch.nn.Linear(in_f, r, bias=False, device=dev)})
        self.lora_B = torch.nn.ModuleDict(
            {adapter: torch.nn.Linear(r, out_f, bias=False, device=dev)})
        torch.nn.init.kaiming_uniform_(self.lora_A[adapter].weight, a=math.sqrt(5))
        if init_b_std:
            torch.nn.init.normal_(self.lora_B[adapter].weight, std=init_b_std)
        else:
            torch.nn.init.zeros_(self.lora_B[adapter].weight)
        self.lora_dropout = torch.nn.ModuleDict(
            {adapter: torch.nn.Dropout(lora_dropout) if lora_dropout > 0 else torch.nn.Identity()})
        self.scaling = {adapter: lora_alpha / r}
        self.r = {adapter: r}
        self.active_adapters = [adapter]
        self.disable_adapters = False
        self.merged = False
        self.compute_dtype = compute_dtype

    @property
    def in_features(self):
        return self.base_layer.in_features

    @property
    def out_features(self):
        return self.base_layer.out_features

    def forward(self, x, *args, **kwargs):
        out = lora_forward(self, x, *args, **kwargs)
        if out is None:
            from . import eager

            return eager.lora_forward_eager(self, x)
        return out


def patch():
    """Route peft's 4-bit LoRA layer through `lora_forward` when peft is importable
    (solution/lora.py:145-176). This package's LoraLinear4bit needs no patch."""
    try:
        from peft.tuners.lora import bnb as lora_bnb
    except ImportError:
        return
    cls = getattr(lora_bnb, "Linear4bit", None)
    if cls is None:
        return
    original = cls.forward
    if getattr(original, "_solution_patch", False):
        return

    def forward(self, x, *args, **kwargs):
        out = lora_forward(self, x, *args, **kwargs)
        return original(self, x, *args, **kwargs) if out is None else out

    forward._solution_patch = True
    cls.forward = forward
