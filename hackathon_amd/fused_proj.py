"""The q/k/v and gate/up projections of a Qwen2 decoder layer as one 4-bit LoRA GEMM each.

In the reference each projection is its own peft 4-bit LoRA layer (solution/lora.py:145-176 over
solution/nf4.py:95-149): q, k and v read the same normalised hidden state, and so do gate and
up. Here each group runs as one fused computation with the same sums:

  forward   u_g = x A_g^T for every projection g            qlora_lora_down, all slots at once
            [y_1 | y_2 | ..] = [x | u] [W_cat | sB_cat]^T + b  qlora_gemm_nt_cat into column ranges
                                                            of one output (W_g dequantised into
                                                            row ranges of one buffer; slot g of
                                                            sB_cat holds s_g B_g in g's rows)
  backward  du_g = s_g dY_g B_g                              qlora_lora_down into slot g (for
                                                            gate/up fused into the SwiGLU
                                                            backward that makes dY_g)
            dx = [dY_1 | dY_2 | .. | du] [W_cat^T | A_cat^T]^T  one GEMM over the concatenated K
            dA_g = du_g^T x                                 qlora_lora_wgrad, all slots at once
            dB_g = s_g dY_g^T u_g                           qlora_lora_wgrad per projection

so the gradient that autograd would otherwise assemble from one dX GEMM per projection plus the
element-wise adds becomes one fp32 accumulation.

With LoRA dropout (p > 0, the same p on every projection of the group) each adapter draws its
own mask of x from its own seed, as the layers one by one do (solution/lora.py:29-46,157-173):

  forward   keep_g as bits, u_g = xd_g A_g^T                 qlora_lora_dropout_down, every
            (xd_g = x * keep_g / (1 - p), never stored)      adapter in one pass over x
            y = [x | u] [W_cat | sB_cat]^T + b               as above
  backward  dx = dY_cat W_cat + sum_g keep_g (du_g A_g)/(1-p)  the GEMM on the base term, then
                                                            qlora_lora_up_masked_add_slots
            dA_g = du_g^T xd_g                              qlora_lora_wgrad_masked, every
                                                            adapter in one pass over x

and du_g, dB_g as above (neither depends on the mask). The attention group also applies RoPE (the q
and k slices of the output feed the rotation kernel directly and its backward writes the
pre-rotation gradients straight into the slices of the gradient buffer), and the MLP group
applies SwiGLU on the two halves of its output (row-strided kernels). Zero columns of the padded
LoRA operands multiply zeros, so every output is the sum the separate layers compute; only the
order of fp32 accumulation differs.

`patch()` installs both on Qwen2Attention.forward and Qwen2MLP.forward; calls whose layers or
inputs the kernels do not take run the forward that was installed before.
"""

from __future__ import annotations

import math

import torch

from . import _common, _lib, adapter_packs, attention, lora, nf4, rope, swiglu
from . import gemm as _gemm

_PAD = 64  # padded LoRA K segment: up to 4 adapters of rank 16


class _Spec:
    """One projection: packed NF4 weight, quant state, frozen bias, adapter scaling."""
    __slots__ = ("packed", "qs", "bias", "scaling", "n", "p")

    def __init__(self, packed, qs, bias, scaling, p=0.0):
        self.packed, self.qs, self.bias, self.scaling = packed, qs, bias, float(scaling)
        self.n = int(qs.shape[0])
        self.p = float(p)  # LoRA dropout probability (0: off)


def lora_spec(layer, x):
    """(_Spec, A, B) of a 4-bit LoRA projection the fused kernels take for input x (rank 16,
    NF4 base, compute dtype = x's dtype, dropout off or drawn from this package's Philox
    stream), else None."""
    if not hasattr(layer, "lora_A") or not hasattr(layer, "base_layer"):
        return None
    if "forward" in getattr(layer, "__dict__", {}):  # an instance-level forward (the eager path)
        return None
    compute_dtype = _common.autocast_dtype() or getattr(layer, "compute_dtype", None)
    if compute_dtype is None or x.dtype != compute_dtype:
        return None
    adapter = lora._single_adapter(layer)
    if adapter is None:
        return None
    drop = layer.lora_dropout[adapter]
    p = float(drop.p) if isinstance(drop, torch.nn.Dropout) and drop.training else 0.0
    fused = lora._fused_base(layer, adapter, x, compute_dtype, p)
    if fused is None:
        return None
    weight, qs, bias = fused
    return (_Spec(weight, qs, bias, layer.scaling[adapter], p), layer.lora_A[adapter].weight,
            layer.lora_B[adapter].weight)


def _offsets(specs):
    offs = [0]
    for s in specs:
        offs.append(offs[-1] + s.n)
    return offs


def _bias_cat(specs, dtype, device):
    """The concatenated biases in the compute dtype (None when no projection has one), cached on
    the first spec's quant state while the bias tensors are unchanged."""
    if all(s.bias is None for s in specs):
        return None
    key = tuple((None if s.bias is None else (s.bias.data_ptr(), s.bias._version)) for s in specs)
    holder = specs[0].qs
    cached = getattr(holder, "_ql_bias_cat", None)
    if cached is not None and cached[0] == key and cached[1].dtype == dtype:
        return cached[1]
    parts = [torch.zeros(s.n, dtype=dtype, device=device) if s.bias is None else
             s.bias.detach().to(dtype) for s in specs]
    cat = torch.cat(parts).contiguous()
    try:
        holder._ql_bias_cat = (key, cat)
    except AttributeError:
        pass
    return cat


def _t_buffer(rows, m, dtype, device):
    """[rows, m] with a row stride that is a multiple of 8 (the transposed LoRA operands)."""
    return torch.empty((rows, (m + 7) // 8 * 8), dtype=dtype, device=device)[:, :m]


_NARROW = 2048  # projections narrower than this share a forward GEMM with their neighbours


def _column_blocks(specs):
    """[(first, last + 1)] projection ranges of the forward GEMMs over the shared output: a
    wide projection gets its own GEMM (its column count then fills the 256-CU tile grid as it
    does alone: 4096 x 3584 is exactly one wave of 256 x 224 tiles, where the 4096 x 4608 of
    q|k|v would be 288 tiles of 256 x 256, two waves), narrow neighbours share one (k|v)."""
    blocks, start, width = [], 0, 0
    for i, s in enumerate(specs):
        if i > start and (width + s.n > _NARROW or s.n > _NARROW or width > _NARROW):
            blocks.append((start, i))
            start, width = i, 0
        width += s.n
    blocks.append((start, len(specs)))
    return blocks


def group_forward(x2, specs, ab, seeds=None):
    """y [M, sum n_g] = x2 W_cat^T + u sB_cat^T + bias, the state the backward needs and, with
    dropout (specs' p > 0, one seed per adapter), (p, a16, [keep bits_g]), else None."""
    dt = x2.dtype
    dev = x2.device
    M, K = x2.shape
    G = len(specs)
    offs = _offsets(specs)
    a16, at, bs, bt = adapter_packs.pack_group(
        [(ab[2 * g], ab[2 * g + 1], specs[g].scaling) for g in range(G)], dt, _PAD)
    u = torch.empty((M, _PAD), dtype=dt, device=dev)
    ut = _t_buffer(16 * G, M, dt, dev)
    drop = None
    p = specs[0].p
    if p > 0 and K % 64 == 0:
        # each adapter's own mask of x (kept as bits) and its u, all adapters in one pass over x
        _, bitss = lora.dropout_down(x2, a16, p, seeds, u, ut)
        drop = (p, a16, bitss)
    elif p > 0:
        # one adapter at a time: slot g's lora_down writes u columns 16 g .. 16 g + 15 and
        # zeros after them, which the later slots overwrite
        bitss = []
        for g in range(G):
            xd, bits = lora.dropout_with_bits(x2, p, seeds[g])
            _gemm.lora_down(xd, a16[16 * g:16 * g + 16], u[:, 16 * g:],
                            out_t=ut[16 * g:16 * g + 16])
            bitss.append(bits)
        drop = (p, a16, bitss)
    else:
        _gemm.lora_down(x2, a16, u, out_t=ut)  # every slot in one pass over x
    y = torch.empty((M, offs[-1]), dtype=dt, device=dev)
    bias = _bias_cat(specs, dt, dev)
    if all(nf4.use_fused_gemm(x2, s.qs, s.packed, a2=u) for s in specs):
        # few rows: each projection's W dequantised inside its GEMM (bs rows of projection g
        # are zero outside slot g, so u's other slots add nothing)
        for g, s in enumerate(specs):
            c0, c1 = offs[g], offs[g + 1]
            nf4.gemm_nf4(x2, s.packed, s.qs, out=y[:, c0:c1], a2=u, b2=bs[c0:c1],
                         bias=None if bias is None else bias[c0:c1])
        return y, (at, bt, ut), drop
    w = torch.empty((offs[-1], K), dtype=dt, device=dev)
    nf4.dequantize_nf4_group([(s.packed, s.qs) for s in specs], dt,
                             [w[offs[g]:offs[g + 1]] for g in range(G)])
    for p0, p1 in _column_blocks(specs):
        c0, c1 = offs[p0], offs[p1]
        _gemm.gemm_nt_cat(x2, w[c0:c1], u, bs[c0:c1], y[:, c0:c1],
                          bias=None if bias is None else bias[c0:c1])
    return y, (at, bt, ut), drop


def group_backward(g, x2, at, bt, ut, specs, need_dx, need_ab, du_dut=None, db_given=None,
                   drop=None):
    """(dx or None, [dA_0, dB_0, dA_1, ...] with None where not needed) for the output
    gradient g [M, sum n_g] (row stride a multiple of 8, unit column stride). `du_dut`, when
    given, holds the adapters' down-projections of g already (du [M, 64], du^T [16 G, M]);
    `db_given`, the lora_B gradients [dB_0, dB_1, ..] already computed; `drop`, group_forward's
    dropout state."""
    dt = g.dtype
    dev = g.device
    M = g.shape[0]
    K = int(specs[0].qs.shape[1])
    G = len(specs)
    offs = _offsets(specs)
    same_scaling = len({s.scaling for s in specs}) == 1
    if du_dut is None:
        du = torch.empty((M, _PAD), dtype=dt, device=dev)
        dut = _t_buffer(16 * G, M, dt, dev)
        if same_scaling:  # bt is block-diagonal: every adapter's du in one pass over g
            _gemm.lora_down(g, bt, du, alpha=specs[0].scaling, out_t=dut)
        else:
            for i, s in enumerate(specs):
                _gemm.lora_down(g[:, offs[i]:offs[i + 1]],
                                bt[16 * i:16 * i + 16, offs[i]:offs[i + 1]], du[:, 16 * i:],
                                alpha=s.scaling, out_t=dut[16 * i:16 * i + 16])
    else:
        du, dut = du_dut
    dx = None
    if need_dx:
        wt = torch.empty((K, offs[-1]), dtype=dt, device=dev)
        nf4.dequantize_nf4_t_group([(s.packed, s.qs) for s in specs], dt,
                                   [wt[:, offs[i]:offs[i + 1]] for i in range(G)])
        dx = torch.empty((M, K), dtype=dt, device=dev)
        if drop is None:
            _gemm.gemm_nt_cat(g, wt, du, at, dx)
        else:
            p, a16, bitss = drop
            _gemm.gemm_nt_cat(g, wt, None, None, dx)
            lora.up_masked_add_slots(dx, du, a16, bitss, p)  # every adapter in one pass
        del wt
    grads = []
    da_all = None
    if drop is not None and any(need_ab[0::2]):
        # dA_g^T = du_g^T xd_g, each adapter on its own dropped input, all in one pass over x
        # (xd_g formed from x and adapter g's keep bits)
        da_all = _gemm.lora_wgrad_masked(dut, x2, drop[2], drop[0])
        da_all = [da_all[16 * i:16 * i + 16] for i in range(G)]
    elif drop is None and any(need_ab[0::2]):  # dA_g^T for every slot in one pass over x
        da_all = _gemm.lora_wgrad(dut, x2, transposed=True)
        da_all = [da_all[16 * i:16 * i + 16] for i in range(G)]
    db_all = None
    if db_given is None and sum(need_ab[1::2]) > 1:  # every dB_g in one pass over g
        db_all = _gemm.lora_wgrad_diag(ut[:16 * G], g, offs, [s.scaling for s in specs])
    for i, s in enumerate(specs):
        da = db = None
        if need_ab[2 * i]:
            da = da_all[i]
        if need_ab[2 * i + 1]:
            if db_given is not None:
                db = db_given[i]
            elif db_all is not None:
                db = db_all[offs[i]:offs[i + 1]]
            else:
                db = _gemm.lora_wgrad(ut[16 * i:16 * i + 16], g[:, offs[i]:offs[i + 1]],
                                      alpha=s.scaling)
        grads += [da, db]
    return dx, grads


def _save(ctx, x2, drop, *tensors):
    """save_for_backward of a group's state: x2, and with dropout a16 and every adapter's keep
    bits (the lora_A gradients form the dropped inputs from x2 and the bits)."""
    if drop is None:
        ctx.save_for_backward(x2, *tensors)
        ctx.n_drop, ctx.p = 0, 0.0
    else:
        p, a16, bitss = drop
        ctx.save_for_backward(x2, a16, *bitss, *tensors)
        ctx.n_drop, ctx.p = len(bitss), p


def _saved(ctx):
    """(x2, dropout state or None, the other saved tensors) as _save stored them."""
    t = ctx.saved_tensors
    G = ctx.n_drop
    if G == 0:
        return t[0], None, t[1:]
    return t[0], (ctx.p, t[1], list(t[2:2 + G])), t[2 + G:]


class QKVRoPE(torch.autograd.Function):
    """x [B, S, K] -> (q, k, v) in the (B, H, S, D) layout of Qwen2Attention: the q/k/v LoRA
    projections as one GEMM, then RoPE on q and k (solution/rope.py:82-104 math). v is a view
    of the projection output. `seeds`: one dropout seed per adapter when the specs' p > 0."""

    @staticmethod
    def forward(ctx, x, cos, sin, hq, hk, specs, seeds, *ab):
        B, S, K = x.shape
        x2 = x.reshape(-1, K)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        y, (at, bt, ut), drop = group_forward(x2, specs, ab, seeds)
        d = specs[0].n // hq
        y4 = y.view(B, S, hq + 2 * hk, d)
        q_pre = y4[:, :, :hq].transpose(1, 2)
        k_pre = y4[:, :, hq:hq + hk].transpose(1, 2)
        v = y4[:, :, hq + hk:].transpose(1, 2)
        cos3 = cos.expand(B, S, -1)
        sin3 = sin.expand(B, S, -1)
        q = torch.empty((B, S, hq, d), dtype=x.dtype, device=x.device).transpose(1, 2)
        k = torch.empty((B, S, hk, d), dtype=x.dtype, device=x.device).transpose(1, 2)
        rope._launch(q_pre, k_pre, cos3, sin3, q, k, backward=False)
        _save(ctx, x2, drop, at, bt, ut, cos3, sin3)
        ctx.specs, ctx.dims = specs, (B, S, K, hq, hk, d)
        ctx.ab_dtypes = [t.dtype for t in ab]
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        x2, drop, (at, bt, ut, cos3, sin3) = _saved(ctx)
        B, S, K, hq, hk, d = ctx.dims
        dt, dev = at.dtype, at.device
        g = torch.empty((B * S, (hq + 2 * hk) * d), dtype=dt, device=dev)
        g4 = g.view(B, S, hq + 2 * hk, d)
        gq = g4[:, :, :hq].transpose(1, 2)
        gk = g4[:, :, hq:hq + hk].transpose(1, 2)
        gv = g4[:, :, hq + hk:].transpose(1, 2)

        def unit(t, h):
            if t is None:
                return torch.zeros((B, h, S, d), dtype=dt, device=dev)
            t = t if t.dtype == dt else t.to(dt)
            return t if t.stride(-1) == 1 else t.contiguous()

        rope._launch(unit(dq, hq), unit(dk, hk), cos3, sin3, gq, gk, backward=True)
        if dv is None:
            gv.zero_()
        else:
            gv.copy_(dv)
        need_ab = ctx.needs_input_grad[7:]
        dx, grads = group_backward(g, x2, at, bt, ut, ctx.specs, ctx.needs_input_grad[0],
                                   need_ab, drop=drop)
        grads = [None if gr is None else gr.to(t) for gr, t in zip(grads, ctx.ab_dtypes)]
        return ((None if dx is None else dx.view(B, S, K)), None, None, None, None, None, None,
                *grads)


class GateUpSwiGLU(torch.autograd.Function):
    """x [.., K] -> silu(gate_proj(x)) * up_proj(x): the two LoRA projections as one GEMM, then
    SwiGLU on the two halves of its output (solution/swiglu.py:15-37 math). `seeds`: one
    dropout seed per adapter when the specs' p > 0."""

    @staticmethod
    def forward(ctx, x, specs, seeds, *ab):
        K = x.shape[-1]
        x2 = x.reshape(-1, K)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        y, (at, bt, ut), drop = group_forward(x2, specs, ab, seeds)
        n = specs[0].n
        h = torch.empty((x2.shape[0], n), dtype=x.dtype, device=x.device)
        swiglu.swiglu_rows(y[:, :n], y[:, n:], h)
        _save(ctx, x2, drop, y, at, bt, ut)
        ctx.specs, ctx.shape = specs, x.shape
        ctx.ab_dtypes = [t.dtype for t in ab]
        return h.view(*x.shape[:-1], n)

    @staticmethod
    def backward(ctx, dh):
        x2, drop, (y, at, bt, ut) = _saved(ctx)
        n = ctx.specs[0].n
        M = y.shape[0]
        dt, dev = y.dtype, y.device
        dh2 = dh.reshape(M, n)
        if dh2.dtype != dt:
            dh2 = dh2.to(dt)
        if dh2.stride(-1) != 1 or dh2.stride(0) % 8 or dh2.data_ptr() % 16:
            dh2 = dh2.contiguous()
        g = torch.empty((M, 2 * n), dtype=dt, device=dev)
        du_dut = db_given = None
        need_ab = ctx.needs_input_grad[3:]
        if n % 32 == 0:
            # the SwiGLU gradients and, in the same pass, du_gate = s dgate B_gate and
            # du_up = s dup B_up, plus (when wanted) both lora_B gradients s dgate^T u_gate and
            # s dup^T u_up: the gradients are not read back from HBM for any of them
            du = torch.empty((M, _PAD), dtype=dt, device=dev)
            dut = _t_buffer(32, M, dt, dev)
            gate_s, up_s = ctx.specs
            if need_ab[1] or need_ab[3]:
                db_given = swiglu.swiglu_bwd_lora(
                    dh2, y[:, :n], y[:, n:], g[:, :n], g[:, n:], bt[:16, :n], bt[16:32, n:], ut[:16],
                    ut[16:32], gate_s.scaling, up_s.scaling, gate_s.scaling, up_s.scaling, du,
                    dut)
            else:
                swiglu.swiglu_bwd_lora_down(dh2, y[:, :n], y[:, n:], g[:, :n], g[:, n:],
                                            bt[:16, :n], bt[16:32, n:], gate_s.scaling, up_s.scaling,
                                            du, dut)
            du_dut = (du, dut)
        else:
            swiglu.swiglu_bwd_rows(dh2, y[:, :n], y[:, n:], g[:, :n], g[:, n:])
        dx, grads = group_backward(g, x2, at, bt, ut, ctx.specs, ctx.needs_input_grad[0],
                                   need_ab, du_dut=du_dut, db_given=db_given, drop=drop)
        grads = [None if gr is None else gr.to(t) for gr, t in zip(grads, ctx.ab_dtypes)]
        return (None if dx is None else dx.view(ctx.shape)), None, None, *grads


class LoraMLP(torch.autograd.Function):
    """x -> down_proj(silu(gate_proj(x)) * up_proj(x)) when all three projections are 4-bit
    LoRA layers: GateUpSwiGLU's gate/up group and the down projection as LoraNF4Linear's two
    GEMMs, with the down adapter's products on h = silu(gate) up fused into the SwiGLU kernels
    (solution/swiglu.py:15-37 and solution/lora.py:157-173 math):

      forward   h and u_d = h A_d^T                        qlora_swiglu_fwd_lora_down
                out = [h | u_d] [W_d | s_d B_d]^T + b_d     qlora_gemm_nt_cat
      backward  du_d = s_d dY B_d                           qlora_lora_down
                dh = [dY | du_d] [W_d^T | A_d^T]^T          qlora_gemm_nt_cat
                dB_d = s_d dY^T u_d                         qlora_lora_wgrad
                dgate, dup, du_gate, du_up, dB_gate, dB_up  qlora_swiglu_bwd_lora, which also
                and dA_d = du_d^T h                         recomputes h on chip for dA_d
                dx, dA_gate, dA_up                          as GateUpSwiGLU

    h is not kept for the backward: it is neither read back for u_d nor stored for dA_d.

    `residual` (None, or [..., N] in x's dtype, contiguous, 16-B aligned) is the decoder
    layer's stream the output is added to (`residual + mlp(x)`, modeling_qwen2.py:297): the
    down GEMM adds it in its store (qlora_gemm_nt_cat_residual, the same two roundings), and
    its gradient is dY itself.

    With LoRA dropout (`seeds`: the gate, up and down adapters' seeds, None where that p is 0)
    the gate/up group drops x per adapter as GateUpSwiGLU does, and the down adapter's input is
    its own mask of h: the forward kernel draws it and keeps it as bits
    (qlora_swiglu_fwd_lora_down_dropout, u_d from the dropped h); in the backward the adapter
    term of dh goes through that mask inside the SwiGLU kernel instead of the GEMM's second K
    segment (the sum qlora_lora_up_masked_add would write, bit for bit), and the kernel drops its
    recomputed h with the same bits for dA_d (qlora_swiglu_bwd_lora_dropout)."""

    @staticmethod
    def forward(ctx, x, specs, dspec, seeds, residual, *ab):
        K = x.shape[-1]
        x2 = x.reshape(-1, K)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        dt, dev = x2.dtype, x2.device
        M = x2.shape[0]
        seeds = seeds or (None, None, None)
        y, (at, bt, ut), drop = group_forward(x2, specs, ab[:4],
                                              seeds[:2] if specs[0].p > 0 else None)
        n, N = specs[0].n, dspec.n
        a16_d, at_d, bs_d, bt_d = adapter_packs.pack(ab[4], ab[5], dspec.scaling, dt, _PAD)
        h = torch.empty((M, n), dtype=dt, device=dev)
        u_d = torch.empty((M, _PAD), dtype=dt, device=dev)
        ut_d = _gemm.lora_t_buffer(M, dt, dev)
        bits_d = swiglu.swiglu_fwd_lora_down(y[:, :n], y[:, n:], h, a16_d, u_d, ut_d,
                                             p=dspec.p, seed=seeds[2] or 0)
        out = torch.empty((M, N), dtype=dt, device=dev)
        bias = None if dspec.bias is None else dspec.bias.to(dt)
        res2 = None if residual is None else residual.view(M, N)
        if nf4.use_fused_gemm(h, dspec.qs, dspec.packed, a2=u_d):  # W_d dequantised in-GEMM
            nf4.gemm_nf4(h, dspec.packed, dspec.qs, out=out, a2=u_d, b2=bs_d, bias=bias)
            if res2 is not None:
                out = res2 + out
        else:
            w = nf4.dequantize_nf4(dspec.packed, dspec.qs, dt)
            if res2 is not None and bias is None:
                _gemm.gemm_nt_cat(h, w, u_d, bs_d, out, residual=res2)
            else:
                _gemm.gemm_nt_cat(h, w, u_d, bs_d, out, bias=bias)
                if res2 is not None:
                    out = res2 + out
            del w
        del h, u_d
        saved = [x2, y, at, bt, ut, at_d, bt_d, ut_d]
        ctx.drop_d = bits_d is not None
        if ctx.drop_d:
            saved += [a16_d, bits_d]
        ctx.n_drop = 0 if drop is None else len(drop[2])
        if drop is not None:
            saved += [drop[1], *drop[2]]
            ctx.p = drop[0]
        ctx.save_for_backward(*saved)
        ctx.specs, ctx.dspec, ctx.shape = specs, dspec, x.shape
        ctx.ab_dtypes = [t.dtype for t in ab]
        return out.view(*x.shape[:-1], N)

    @staticmethod
    def backward(ctx, dout):
        t = list(ctx.saved_tensors)
        x2, y, at, bt, ut, at_d, bt_d, ut_d = t[:8]
        t = t[8:]
        a16_d = bits_d = None
        if ctx.drop_d:
            a16_d, bits_d = t[:2]
            t = t[2:]
        drop = None if ctx.n_drop == 0 else (ctx.p, t[0], t[1:1 + ctx.n_drop])
        specs, dspec = ctx.specs, ctx.dspec
        dt, dev = x2.dtype, x2.device
        M = x2.shape[0]
        n, N = specs[0].n, dspec.n
        # x, specs, dspec, seeds, residual, A_gate, B_gate, A_up, B_up, A_d, B_d
        need = ctx.needs_input_grad
        dres = dout if need[4] else None
        dy = dout.reshape(M, N)
        if dy.dtype != dt:
            dy = dy.to(dt)
        if dy.stride(-1) != 1 or dy.stride(0) % 8 or dy.data_ptr() % 16:
            dy = dy.contiguous()
        s_d = dspec.scaling
        du_d = torch.empty((M, _PAD), dtype=dt, device=dev)
        dut_d = _gemm.lora_t_buffer(M, dt, dev)
        _gemm.lora_down(dy, bt_d, du_d, alpha=s_d, out_t=dut_d)  # du_d = s_d dY B_d
        wt = nf4.dequantize_nf4_t(dspec.packed, dspec.qs, dt)    # W_d^T [n, N]
        dh = torch.empty((M, n), dtype=dt, device=dev)
        if bits_d is None:
            _gemm.gemm_nt_cat(dy, wt, du_d, at_d, dh)
        else:  # the adapter term goes through its mask of h inside the SwiGLU backward
            _gemm.gemm_nt_cat(dy, wt, None, None, dh)
        del wt
        db_d = _gemm.lora_wgrad(ut_d, dy, alpha=s_d) if need[10] else None
        g = torch.empty((M, 2 * n), dtype=dt, device=dev)
        du = torch.empty((M, _PAD), dtype=dt, device=dev)
        dut = _t_buffer(32, M, dt, dev)
        gate_s, up_s = specs
        db_g, db_u, da_d = swiglu.swiglu_bwd_lora(
            dh, y[:, :n], y[:, n:], g[:, :n], g[:, n:], bt[:16, :n], bt[16:32, n:], ut[:16], ut[16:32],
            gate_s.scaling, up_s.scaling, gate_s.scaling, up_s.scaling, du, dut, ud_t=dut_d,
            bits_down=bits_d, p_down=dspec.p,
            du_add=None if bits_d is None else du_d, a_add=None if bits_d is None else a16_d)
        del dh, du_d
        dx, grads = group_backward(g, x2, at, bt, ut, specs, need[0], need[5:9],
                                   du_dut=(du, dut), db_given=[db_g, db_u], drop=drop)
        grads = grads + [da_d if need[9] else None, db_d]
        grads = [None if gr is None else gr.to(t_) for gr, t_ in zip(grads, ctx.ab_dtypes)]
        return (None if dx is None else dx.view(ctx.shape)), None, None, None, dres, *grads


def _group(layers, x):
    """(specs, [A_0, B_0, ...]) when every layer of the group is a fused-kernel 4-bit LoRA
    projection of the same input width, else None."""
    specs, ab = [], []
    K = x.shape[-1]
    for layer in layers:
        got = lora_spec(layer, x)
        if got is None:
            return None
        spec, a, b = got
        if int(spec.qs.shape[1]) != K:
            return None
        specs.append(spec)
        ab += [a, b]
    if len({s.p for s in specs}) > 1:  # the group's dropout state takes one p
        return None
    return specs, ab


def _seeds(specs):
    """One dropout seed per adapter, drawn in projection order from the stream the layers one
    by one draw from, or None with dropout off."""
    return tuple(lora._Seeds.next() for _ in specs) if specs[0].p > 0 else None


def _rows_ok(x):
    return (_common.on_gpu(x) and x.dtype in (torch.bfloat16, torch.float16) and x.dim() == 3
            and x.is_contiguous() and x.shape[-1] % 128 == 0 and x.data_ptr() % 16 == 0)


def fused_attention(module, hidden_states, position_embeddings, attention_mask,
                    past_key_values, kwargs):
    """Qwen2Attention.forward on QKVRoPE + the flash kernels + o_proj, or None when this call
    must take the installed forward."""
    cfg = module.config
    if past_key_values is not None or attention_mask is not None or position_embeddings is None:
        return None
    if getattr(cfg, "_attn_implementation", None) != "sdpa":
        return None
    if kwargs.get("output_attentions", False) or getattr(module, "sliding_window", None):
        return None
    if module.training and module.attention_dropout:
        return None
    if not _rows_ok(hidden_states):
        return None
    hq, hk = cfg.num_attention_heads, cfg.num_key_value_heads
    d = module.head_dim
    if d != attention.HEAD_DIM or hq % hk:
        return None
    cos, sin = position_embeddings
    B, S, _ = hidden_states.shape
    if (cos.dtype != hidden_states.dtype or sin.dtype != cos.dtype or cos.dim() != 3
            or cos.shape[-2:] != (S, d) or cos.shape[0] not in (1, B) or sin.shape != cos.shape
            or not _common.on_gpu(cos, sin) or cos.requires_grad or sin.requires_grad):
        return None
    group = _group((module.q_proj, module.k_proj, module.v_proj), hidden_states)
    if group is None:
        return None
    specs, ab = group
    if [s.n for s in specs] != [hq * d, hk * d, hk * d]:
        return None
    cos = cos if cos.stride(-1) == 1 else cos.contiguous()
    sin = sin if sin.stride(-1) == 1 else sin.contiguous()
    q, k, v = QKVRoPE.apply(hidden_states, cos, sin, hq, hk, tuple(specs), _seeds(specs), *ab)
    scale = getattr(module, "scaling", 1.0 / math.sqrt(d))
    attn = attention.flash_attention(q, k, v, scale)  # [B, S, HQ, D]
    return module.o_proj(attn.reshape(B, S, -1)), None


def _residual_ok(residual, x, N):
    return (residual.dtype == x.dtype and residual.shape == (*x.shape[:-1], N)
            and residual.is_contiguous() and residual.data_ptr() % 16 == 0 and N % 8 == 0
            and residual.device == x.device)


def fused_mlp(module, x, residual=None):
    """Qwen2MLP.forward as LoraMLP(x) when the down projection is a fused-kernel 4-bit LoRA
    layer too, else down_proj(GateUpSwiGLU(x)); None when the gate/up group does not fit.
    With `residual`: residual + that output (the decoder layer's last add), taken into the
    down GEMM when LoraMLP can."""
    if getattr(getattr(module, "config", None), "hidden_act", "silu") != "silu":
        return None
    if not (_common.on_gpu(x) and x.dtype in (torch.bfloat16, torch.float16)
            and x.is_contiguous() and x.data_ptr() % 16 == 0):
        return None
    group = _group((module.gate_proj, module.up_proj), x)
    if group is None:
        return None
    specs, ab = group
    n = specs[0].n
    if specs[1].n != n or n % 8:
        return None
    down = lora_spec(module.down_proj, x) if n % 32 == 0 else None
    if down is not None and int(down[0].qs.shape[1]) == n:
        dspec, a_d, b_d = down
        # the layers one by one draw their seeds in this order: gate, up, down
        seeds = _seeds(specs) or (None, None)
        seeds = seeds + ((lora._Seeds.next() if dspec.p > 0 else None),)
        if all(s_ is None for s_ in seeds):
            seeds = None
        if residual is not None and not _residual_ok(residual, x, dspec.n):
            return residual + LoraMLP.apply(x, tuple(specs), dspec, seeds, None, *ab, a_d, b_d)
        return LoraMLP.apply(x, tuple(specs), dspec, seeds, residual, *ab, a_d, b_d)
    out = module.down_proj(GateUpSwiGLU.apply(x, tuple(specs), _seeds(specs), *ab))
    return out if residual is None else residual + out


def patch():
    """Install the fused q/k/v and gate/up forwards on Qwen2Attention and Qwen2MLP (each
    falling back to the forward installed before it)."""
    from transformers.models.qwen2 import modeling_qwen2 as m

    attn_prev = m.Qwen2Attention.forward
    if not getattr(attn_prev, "_solution_fused_proj", False):
        def attn_forward(self, hidden_states, position_embeddings=None, attention_mask=None,
                         past_key_values=None, **kwargs):
            out = fused_attention(self, hidden_states, position_embeddings, attention_mask,
                                  past_key_values, kwargs)
            if out is None:
                return attn_prev(self, hidden_states, position_embeddings, attention_mask,
                                 past_key_values=past_key_values, **kwargs)
            return out

        attn_forward._solution_patch = True
        attn_forward._solution_fused_proj = True
        attn_forward._original = attn_prev
        m.Qwen2Attention.forward = attn_forward

    mlp_prev = m.Qwen2MLP.forward
    if not getattr(mlp_prev, "_solution_fused_proj", False):
        def mlp_forward(self, x):
            out = fused_mlp(self, x)
            return mlp_prev(self, x) if out is None else out

        mlp_forward._solution_patch = True
        mlp_forward._solution_fused_proj = True
        mlp_forward._original = mlp_prev
        m.Qwen2MLP.forward = mlp_forward
