"""Host logic of the decoder layer's fused last add (no GPU): when the MLP's call may take the
residual, and which residuals the down GEMM's store accepts."""

import torch

from hackathon_amd import fused_proj, residual


def test_plain_call_sees_module_and_global_hooks():
    m = torch.nn.Linear(8, 8)
    assert residual._plain_call(m)
    h = m.register_forward_pre_hook(lambda mod, inp: None)
    assert not residual._plain_call(m)
    h.remove()
    assert residual._plain_call(m)
    g = torch.nn.modules.module.register_module_forward_hook(lambda mod, inp, out: None)
    try:
        assert not residual._plain_call(m)
    finally:
        g.remove()
    m.forward = lambda x: x          # a forward set on the instance
    assert not residual._plain_call(m)


def test_an_unpatched_mlp_keeps_the_plain_add():
    m = torch.nn.Linear(8, 8)        # its forward is not the fused MLP forward
    assert residual._mlp_with_residual(m, torch.zeros(2, 8), torch.zeros(2, 8)) is None


def test_residual_accepted_only_as_the_store_reads_it():
    x = torch.zeros(2, 4, 64, dtype=torch.bfloat16)
    ok = torch.zeros(2, 4, 32, dtype=torch.bfloat16)
    assert fused_proj._residual_ok(ok, x, 32)
    assert not fused_proj._residual_ok(ok.float(), x, 32)                 # another dtype
    assert not fused_proj._residual_ok(ok, x, 40)                         # another width
    wide = torch.zeros(2, 4, 40, dtype=torch.bfloat16)
    assert not fused_proj._residual_ok(wide[..., :32], x, 32)             # not contiguous
    flat = torch.zeros(2 * 4 * 32 + 1, dtype=torch.bfloat16)
    assert not fused_proj._residual_ok(flat[1:].view(2, 4, 32), x, 32)    # not 16-B aligned
    odd = torch.zeros(2, 4, 36, dtype=torch.bfloat16)
    assert not fused_proj._residual_ok(odd, x, 36)                        # rows not 8-aligned
