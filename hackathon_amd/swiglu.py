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


def swiglu_bwd_lora_down(grad, gate, up, dgate, dup, bt_gate, bt_up, alpha_gate, alpha_up,
                         du, du_t=None):
    """The SwiGLU gradients into dgate / dup (as swiglu_bwd_rows) and, in the same pass, the
    gate and up adapters' down-projections of them: du[:, :16] = alpha_gate dgate bt_gate^T,
    du[:, 16:32] = alpha_up dup bt_up^T, du[:, 32:] = 0, du_t = du[:, :32]^T when given
    (qlora_swiglu_bwd_lora_down)."""
    _lib.require_rows(gate.dtype, grad=grad, gate=gate, up=up, dgate=dgate, dup=dup,
                      bt_gate=bt_gate, bt_up=bt_up, du=du, du_t=du_t)
    rows, cols = gate.shape
    if bt_up.stride(0) != bt_gate.stride(0):
        raise ValueError("bt_gate and bt_up must share a row stride (slices of one B^T buffer)")
    ws, ws_bytes = _lib.workspace("qlora_swiglu_bwd_lora_down_workspace_size", rows, cols,
                                  device=gate.device)
    _lib.call("qlora_swiglu_bwd_lora_down", grad.data_ptr(), grad.stride(0), gate.data_ptr(),
              gate.stride(0), up.data_ptr(), up.stride(0), dgate.data_ptr(), dgate.stride(0),
              dup.data_ptr(), dup.stride(0), rows, cols, bt_gate.data_ptr(), bt_up.data_ptr(),
              bt_gate.stride(0), float(alpha_gate), float(alpha_up), _lib.tag(gate.dtype),
              du.data_ptr(), du.stride(0), du.shape[1], _lib.ptr(du_t),
              du_t.stride(0) if du_t is not None else 0, _lib.ptr(ws), ws_bytes,
              _lib.stream_of(gate))


def swiglu_bwd_lora(grad, gate, up, dgate, dup, bt_gate, bt_up, ut_gate, ut_up, alpha_gate,
                    alpha_up, beta_gate, beta_up, du, du_t=None, ud_t=None, beta_down=1.0,
                    bits_down=None, p_down=0.0, du_add=None, a_add=None):
    """swiglu_bwd_lora_down plus both adapters' lora_B gradients in the same pass
    (qlora_swiglu_bwd_lora): returns fp32 (db_gate, db_up) [cols, 16] with
    db_gate = beta_gate dgate^T ut_gate^T and db_up = beta_up dup^T ut_up^T, where ut_* [16, rows]
    are the adapters' down-projections of the forward input, transposed. With `ud_t` (the du^T
    [16, rows] of the adapter of the layer that reads h = silu(gate) up) also that adapter's
    lora_A gradient da_down = beta_down ud_t h [16, cols], h recomputed on chip: returns
    (db_gate, db_up, da_down). With `bits_down` (swiglu_fwd_lora_down's keep bits for dropout
    p_down) h in that product is the adapter's dropped input (qlora_swiglu_bwd_lora_dropout),
    and with `du_add` [rows, >= 16] and `a_add` [16, cols] (that adapter's du and A) the
    gradient differentiated is grad plus that adapter's masked input gradient, the sum
    lora.up_masked_add would leave in grad (grad itself is not written)."""
    _lib.require_rows(gate.dtype, grad=grad, gate=gate, up=up, dgate=dgate, dup=dup,
                      bt_gate=bt_gate, bt_up=bt_up, ut_gate=ut_gate, ut_up=ut_up, du=du,
                      du_t=du_t, ud_t=ud_t)
    rows, cols = gate.shape
    if bt_up.stride(0) != bt_gate.stride(0):
        raise ValueError("bt_gate and bt_up must share a row stride (slices of one B^T buffer)")
    if ut_up.stride(0) != ut_gate.stride(0) or (ud_t is not None
                                                 and ud_t.stride(0) != ut_gate.stride(0)):
        raise ValueError("ut_gate, ut_up and ud_t must share a row stride")
    dev = gate.device
    db_gate = torch.empty((cols, 16), dtype=torch.float32, device=dev)
    db_up = torch.empty((cols, 16), dtype=torch.float32, device=dev)
    da_down = None if ud_t is None else torch.empty((16, cols), dtype=torch.float32, device=dev)
    ws, ws_bytes = _lib.workspace("qlora_swiglu_bwd_lora_workspace_size", rows, cols,
                                  int(ud_t is not None), device=dev)
    args = (grad.data_ptr(), grad.stride(0), gate.data_ptr(), gate.stride(0), up.data_ptr(),
            up.stride(0), dgate.data_ptr(), dgate.stride(0), dup.data_ptr(), dup.stride(0), rows,
            cols, bt_gate.data_ptr(), bt_up.data_ptr(), bt_gate.stride(0), ut_gate.data_ptr(),
            ut_up.data_ptr(), ut_gate.stride(0), float(alpha_gate), float(alpha_up),
            float(beta_gate), float(beta_up), _lib.tag(gate.dtype), du.data_ptr(), du.stride(0),
            du.shape[1], _lib.ptr(du_t), du_t.stride(0) if du_t is not None else 0,
            db_gate.data_ptr(), db_up.data_ptr(), _lib.ptr(ud_t), float(beta_down),
            _lib.ptr(da_down))
    if bits_down is None:
        _lib.call("qlora_swiglu_bwd_lora", *args, _lib.ptr(ws), ws_bytes, _lib.stream_of(gate))
    else:
        if du_add is not None:
            _lib.require_rows(gate.dtype, du_add=du_add, a_add=a_add)
        _lib.call("qlora_swiglu_bwd_lora_dropout", *args, bits_down.data_ptr(),
                  bits_down.stride(0), float(p_down), 1.0 / (1.0 - p_down), _lib.ptr(du_add),
                  du_add.stride(0) if du_add is not None else 0, _lib.ptr(a_add),
                  a_add.stride(0) if a_add is not None else 0, _lib.ptr(ws), ws_bytes,
                  _lib.stream_of(gate))
    return (db_gate, db_up) if ud_t is None else (db_gate, db_up, da_down)


def swiglu_fwd_lora_down(gate, up, h, a, u, u_t=None, alpha=1.0, p=0.0, seed=0):
    """h = silu(gate) * up (as swiglu_rows) and, in the same pass, the down-projection of h by
    the next layer's adapter: u[:, :16] = alpha h a^T for a [16, cols] (that adapter's A in the
    compute dtype), u[:, 16:] = 0, u_t = u[:, :16]^T when given (qlora_swiglu_fwd_lora_down).
    With dropout p > 0 that adapter's input is its own mask of h (Philox seed `seed`): u is
    taken on the dropped h and the keep bits are returned (lora.keep_bits_buffer's layout;
    qlora_swiglu_fwd_lora_down_dropout), else None."""
    from . import lora

    _lib.require_rows(gate.dtype, gate=gate, up=up, h=h, a=a, u=u, u_t=u_t)
    rows, cols = gate.shape
    ws, ws_bytes = _lib.workspace("qlora_swiglu_fwd_lora_down_workspace_size", rows, cols,
                                  device=gate.device)
    args = (gate.data_ptr(), gate.stride(0), up.data_ptr(), up.stride(0), h.data_ptr(),
            h.stride(0), rows, cols, a.data_ptr(), a.stride(0), float(alpha), _lib.tag(gate.dtype),
            u.data_ptr(), u.stride(0), u.shape[1], _lib.ptr(u_t),
            u_t.stride(0) if u_t is not None else 0)
    if p == 0:
        _lib.call("qlora_swiglu_fwd_lora_down", *args, _lib.ptr(ws), ws_bytes,
                  _lib.stream_of(gate))
        return None
    bits = lora.keep_bits_buffer(rows, cols, gate.device)
    _lib.call("qlora_swiglu_fwd_lora_down_dropout", *args, int(seed) & 0xFFFF_FFFF_FFFF_FFFF,
              float(p), 1.0 / (1.0 - p), bits.data_ptr(), bits.stride(0), _lib.ptr(ws), ws_bytes,
              _lib.stream_of(gate))
    return bits


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
