"""Causal attention of the QLoRA step on the gfx950 flash-attention kernels.

The reference leaves attention to torch's scaled_dot_product_attention, which transformers'
Qwen2Attention reaches through `ALL_ATTENTION_FUNCTIONS["sdpa"]`
(transformers/models/qwen2/modeling_qwen2.py:216-229,
transformers/integrations/sdpa_attention.py:79-166). `patch()` wraps that entry: causal
self-attention with no mask, no dropout, head_dim 128 and 16-bit q/k/v on a GPU runs
`FlashAttention` (qlora_attn_fwd, plus the backward kernels); anything else goes to the
original function unchanged.
"""

from __future__ import annotations

import math

import torch

from . import _common, _lib

HEAD_DIM = 128


def _strides3(t):
    return _lib.i64_array([t.stride(0), t.stride(1), t.stride(2)])


def attn_fwd(q, k, v, scale, with_lse=True):
    """(o [B, S, HQ, D] contiguous, lse fp32 [B, HQ, S]) for q [B, HQ, S, D] and k, v
    [B, HK, S, D] (any strides with a unit last dim)."""
    _lib.require_device(q, k, v)
    B, HQ, S, D = q.shape
    HK = k.shape[1]
    o = torch.empty((B, S, HQ, D), dtype=q.dtype, device=q.device)
    ov = o.transpose(1, 2)  # (B, HQ, S, D) view with BSHD storage
    lse = torch.empty((B, HQ, S), dtype=torch.float32, device=q.device) if with_lse else None
    _lib.call("qlora_attn_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
              _lib.ptr(lse), _lib.tag(q.dtype), B, HQ, HK, S, D, _strides3(q), _strides3(k),
              _strides3(v), _strides3(ov), float(scale), _lib.stream_of(q))
    return o, lse


def attn_bwd(q, k, v, o, lse, do, scale):
    """(dq, dk, dv) in the layouts of q, k and v as (B, H, S, D) views of (B, S, H, D) storage,
    for the forward `attn_fwd(q, k, v, scale)` = (o, lse) and the output gradient `do`."""
    _lib.require_device(q, k, v, o, do)
    B, HQ, S, D = q.shape
    HK = k.shape[1]
    if do.stride() != o.stride():
        do = do.contiguous()
    dq = torch.empty((B, S, HQ, D), dtype=q.dtype, device=q.device).transpose(1, 2)
    dk = torch.empty((B, S, HK, D), dtype=q.dtype, device=q.device).transpose(1, 2)
    dv = torch.empty((B, S, HK, D), dtype=q.dtype, device=q.device).transpose(1, 2)
    ws, ws_bytes = _lib.workspace("qlora_attn_bwd_workspace_size", B, HQ, HK, S,
                                  device=q.device)
    _lib.call("qlora_attn_bwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
              do.data_ptr(), lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
              _lib.tag(q.dtype), B, HQ, HK, S, D, _strides3(q), _strides3(k), _strides3(v),
              _strides3(o.transpose(1, 2)), _strides3(dq), _strides3(dk), float(scale),
              _lib.ptr(ws), ws_bytes, _lib.stream_of(q))
    return dq, dk, dv


class FlashAttention(torch.autograd.Function):
    """Causal attention o [B, S, HQ, D] = softmax(scale q k^T) v for q [B, HQ, S, D] and k, v
    [B, HK, S, D] (grouped-query heads), as the SDPA path computes it, on the flash kernels."""

    @staticmethod
    def forward(ctx, q, k, v, scale):
        o, lse = attn_fwd(q, k, v, scale, with_lse=True)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale = scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = attn_bwd(q, k, v, o, lse, do, ctx.scale)
        return dq, dk, dv, None


def flash_attention(q, k, v, scale=None):
    """Causal attention on the flash kernels: o [B, S, HQ, D] (the layout transformers' SDPA
    integration returns) for q [B, HQ, S, D] and k, v [B, HK, S, D]."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    return FlashAttention.apply(q, k, v, float(scale))


def supported(module, query, key, value, attention_mask, dropout, is_causal, kwargs):
    """Whether a transformers attention call can take the flash kernels."""
    if not _common.on_gpu(query, key, value) or attention_mask is not None or dropout:
        return False
    if is_causal is False or (is_causal is None and not getattr(module, "is_causal", True)):
        return False
    if kwargs.get("output_attentions", False) or kwargs.get("position_bias") is not None:
        return False
    if kwargs.get("sliding_window") is not None:
        return False
    if query.dtype not in (torch.bfloat16, torch.float16) or key.dtype != query.dtype \
            or value.dtype != query.dtype:
        return False
    if query.shape[-1] != HEAD_DIM or key.shape[-1] != HEAD_DIM or value.shape[-1] != HEAD_DIM:
        return False
    if query.shape[2] != key.shape[2] or query.shape[1] % key.shape[1]:
        return False
    return all(t.stride(-1) == 1 and all(s % 8 == 0 for s in t.stride()[:3])
               and t.data_ptr() % 16 == 0 for t in (query, key, value))


def patch():
    """Route transformers' "sdpa" attention through `flash_attention` for the calls `supported`
    accepts; every other call goes to the original function unchanged."""
    from transformers.modeling_utils import AttentionInterface

    original = AttentionInterface._global_mapping["sdpa"]
    if getattr(original, "_solution_patch", False):
        return

    def sdpa_attention_forward(module, query, key, value, attention_mask, dropout=0.0,
                               scaling=None, is_causal=None, **kwargs):
        if not supported(module, query, key, value, attention_mask, dropout, is_causal, kwargs):
            return original(module, query, key, value, attention_mask, dropout=dropout,
                            scaling=scaling, is_causal=is_causal, **kwargs)
        return flash_attention(query, key, value, scaling), None

    sdpa_attention_forward._solution_patch = True
    sdpa_attention_forward._original = original
    AttentionInterface._global_mapping["sdpa"] = sdpa_attention_forward
