"""Fused SwiGLU, silu(gate) * up, for the Qwen2 MLP, forward and backward
(drop-in for solution/swiglu.py).

    out   = gate * sigmoid(gate) * up                       (fp32 math, solution/swiglu.py:15-22)
    dup   = g * gate * sig;  dgate = g * up * sig * (1 + gate * (1 - sig))   (:25-37)
"""

from __future__ import annotations

import torch

from . import _lib

BLOCK = 1024  # elements per program in the reference (solution/swiglu.py:12)


class SwiGLU(torch.autograd.Function):
    """solution/swiglu.py:40-61 on `qlora_swiglu_fwd` / `qlora_swiglu_bwd`."""

    @staticmethod
    def forward(ctx, gate, up):
        _lib.require_device(gate, up)
        gate = gate.contiguous()
        up = up.to(gate.dtype).contiguous()
        out = torch.empty_like(gate)
        _lib.call("qlora_swiglu_fwd", gate.data_ptr(), up.data_ptr(), out.data_ptr(),
                  _lib.tag(gate.dtype), gate.numel(), _lib.stream_of(gate))
        ctx.save_for_backward(gate, up)
        return out

    @staticmethod
    def backward(ctx, grad):
        gate, up = ctx.saved_tensors
        grad = grad.to(gate.dtype).contiguous()
        dgate, dup = torch.empty_like(gate), torch.empty_like(up)
        _lib.call("qlora_swiglu_bwd", grad.data_ptr(), gate.data_ptr(), up.data_ptr(),
                  dgate.data_ptr(), dup.data_ptr(), _lib.tag(gate.dtype), gate.numel(),
                  _lib.stream_of(gate))
        return dgate, dup


def swiglu(gate, up):
    return SwiGLU.apply(gate, up)


def swiglu_rows(gate, up, out):
    """out = silu(gate) * up for [rows, cols] operands with their own row strides
    (qlora_swiglu_fwd_rows): gate and up may be column ranges of one buffer."""
    rows, cols = gate.shape
    _lib.call("qlora_swiglu_fwd_rows", gate.data_ptr(), gate.stride(0), up.data_ptr(),
              up.stride(0), out.data_ptr(), out.stride(0), rows, cols, _lib.tag(gate.dtype),
              _lib.stream_of(gate))
    return out


def swiglu_bwd_rows(grad, gate, up, dgate, dup):
    """The SwiGLU gradients into dgate / dup for row-strided operands (qlora_swiglu_bwd_rows)."""
    rows, cols = gate.shape
    _lib.call("qlora_swiglu_bwd_rows", grad.data_ptr(), grad.stride(0), gate.data_ptr(),
              gate.stride(0), up.data_ptr(), up.stride(0), dgate.data_ptr(), dgate.stride(0),
              dup.data_ptr(), dup.stride(0), rows, cols, _lib.tag(gate.dtype),
              _lib.stream_of(gate))


def patch_qwen2_mlp():
    """Send Qwen2MLP.forward through the fused kernel for GPU inputs (solution/swiglu.py:68-81)."""
    from transformers.models.qwen2 import modeling_qwen2

    original = modeling_qwen2.Qwen2MLP.forward
    if getattr(original, "_solution_patch", False):
        return

    def forward(self, x):
        act = getattr(getattr(self, "config", None), "hidden_act", "silu")
        if act != "silu" or not x.is_cuda:
            return original(self, x)
        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x)))

    forward._solution_patch = True
    forward._original = original
    modeling_qwen2.Qwen2MLP.forward = forward
