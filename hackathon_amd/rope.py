"""Rotary position embedding for q and k in one launch, forward and backward
(drop-in for solution/rope.py).

Original (modeling_qwen2.apply_rotary_pos_emb, unsqueeze_dim=1):
    q_out = q*cos + rotate_half(q)*sin,   rotate_half(x) = cat(-x2, x1)
With halves (x1, x2), (c1, c2), (s1, s2) (solution/rope.py:3-15):
    forward:  o1 = x1*c1 - x2*s1          o2 = x2*c2 + x1*s2
    backward: d1 = g1*c1 + g2*s2          d2 = g2*c2 - g1*s1
q and k come in as (B, H, S, D) views of (B, S, H, D) buffers; the kernel takes real strides
and the outputs keep the inputs' layout (empty_like keeps strides). Only cos/sin are saved.
"""

from __future__ import annotations

import torch

from . import _common, _lib


def _strides(t):
    return _lib.i64_array((t.stride(0), t.stride(1), t.stride(2)))


def _launch(q, k, cos, sin, q_out, k_out, backward):
    """One kernel launch for q and k when they share a dtype (solution/rope.py:65-75)."""
    B, HQ, S, D = q.shape
    HK = k.shape[1]
    if sin.dtype != cos.dtype:
        sin = sin.to(cos.dtype)
    groups = [(q, k, q_out, k_out, HQ, HK)] if q.dtype == k.dtype and q_out.dtype == k_out.dtype \
        else [(q, q, q_out, q_out, HQ, 0), (k, k, k_out, k_out, 0, HK)]
    for qq, kk, qo, ko, hq, hk in groups:
        ref = qq if hq else kk
        _lib.call("qlora_rope_qk", qq.data_ptr(), kk.data_ptr(), qo.data_ptr(), ko.data_ptr(),
                  cos.data_ptr(), sin.data_ptr(), _lib.tag(ref.dtype), _lib.tag(cos.dtype),
                  _lib.tag((qo if hq else ko).dtype), B, S, hq, hk, D, _strides(qq),
                  _strides(kk), _strides(qo), _strides(ko), cos.stride(0), cos.stride(1),
                  int(backward), _lib.stream_of(ref))


def _unit_last(t):
    return t if t.stride(-1) == 1 else t.contiguous()


class HipRoPE(torch.autograd.Function):
    """solution/rope.py:82-104 on `qlora_rope_qk`."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        _lib.require_device(q, k, cos, sin)
        B, _, S, _ = q.shape
        q, k = _unit_last(q), _unit_last(k)
        cos = _unit_last(cos).expand(B, S, -1)
        sin = _unit_last(sin).expand(B, S, -1)
        q_out = torch.empty_like(q, dtype=torch.promote_types(q.dtype, cos.dtype))
        k_out = torch.empty_like(k, dtype=torch.promote_types(k.dtype, cos.dtype))
        _launch(q, k, cos, sin, q_out, k_out, backward=False)
        ctx.save_for_backward(cos, sin)
        ctx.q_dtype, ctx.k_dtype = q.dtype, k.dtype
        return q_out, k_out

    @staticmethod
    def backward(ctx, dq_out, dk_out):
        cos, sin = ctx.saved_tensors
        dq_out, dk_out = _unit_last(dq_out), _unit_last(dk_out)
        dq = torch.empty_like(dq_out, dtype=torch.promote_types(dq_out.dtype, cos.dtype))
        dk = torch.empty_like(dk_out, dtype=torch.promote_types(dk_out.dtype, cos.dtype))
        _launch(dq_out, dk_out, cos, sin, dq, dk, backward=True)
        if dq.dtype != ctx.q_dtype:
            dq = dq.to(ctx.q_dtype)
        if dk.dtype != ctx.k_dtype:
            dk = dk.to(ctx.k_dtype)
        return dq, dk, None, None


TritonRoPE = HipRoPE        # the reference's class name (solution/rope.py:82)
RoPEFunction = HipRoPE      # the name solution/test_kernels.py:79 imports


def _supported(q, k, cos, sin, unsqueeze_dim):
    """The shapes the kernel takes (solution/rope.py:107-117)."""
    if not _common.on_gpu(q, k, cos, sin) or unsqueeze_dim != 1:
        return False
    if q.dim() != 4 or k.dim() != 4 or cos.dim() != 3 or sin.shape != cos.shape:
        return False
    B, _, S, D = q.shape
    if k.shape[0] != B or k.shape[2] != S or k.shape[3] != D or D % 2 or (D & (D - 1)):
        return False
    if cos.shape[0] not in (1, B) or cos.shape[1] != S or cos.shape[2] != D:
        return False
    return not (cos.requires_grad or sin.requires_grad)


def patch():
    """Route modeling_qwen2.apply_rotary_pos_emb through HipRoPE (solution/rope.py:120-135)."""
    from transformers.models.qwen2 import modeling_qwen2 as m

    original = m.apply_rotary_pos_emb
    if getattr(original, "_solution_patch", False):
        return

    def apply_rotary_pos_emb(q, k, cos, sin, *args, **kwargs):
        unsqueeze_dim = kwargs.get("unsqueeze_dim", args[0] if args else 1)
        if len(args) > 1 or set(kwargs) - {"unsqueeze_dim"} or \
                not _supported(q, k, cos, sin, unsqueeze_dim):
            return original(q, k, cos, sin, *args, **kwargs)
        return HipRoPE.apply(q, k, cos, sin)

    apply_rotary_pos_emb._solution_patch = True
    apply_rotary_pos_emb._original = original
    m.apply_rotary_pos_emb = apply_rotary_pos_emb
