"""RMSNorm fused with the decoder layer's residual stream.

ResidualRMSNorm against the unfused computation it replaces: h = x + delta bit-identical to
torch's 16-bit add, y bit-identical to the RMSNorm kernel on h; the backward (one fp32 sum of
the two gradients, rounded once) within one bf16 rounding of autograd's rounded-then-added
result (rtol 8e-3) and within 2e-2 of an fp32 reference. The patched Qwen2DecoderLayer: output
bit-identical to the original forward under the same kernels, input gradient within bf16
tolerance of it and of an fp32 copy of the layer run unpatched."""

import copy

import pytest
import torch

import hackathon_amd
from hackathon_amd import qlora_step
from hackathon_amd.residual import residual_rmsnorm
from hackathon_amd.rmsnorm import rmsnorm

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,with_delta", [(64, 3584, True), (37, 1536, True), (64, 3584, False),
                                            (5, 8, True)])
def test_residual_rmsnorm_matches_unfused(M, N, with_delta):
    print(f"residual rmsnorm M={M} N={N} delta={with_delta}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M + N)
    x = torch.randn(M, N, device="cuda", generator=g).to(torch.bfloat16)
    d = torch.randn(M, N, device="cuda", generator=g).to(torch.bfloat16) if with_delta else None
    w = (1 + 0.1 * torch.randn(N, device="cuda", generator=g)).to(torch.bfloat16)
    dh = torch.randn(M, N, device="cuda", generator=g).to(torch.bfloat16)
    dy = torch.randn(M, N, device="cuda", generator=g).to(torch.bfloat16)
    eps = 1e-6

    xf = x.clone().requires_grad_(True)
    df = d.clone().requires_grad_(True) if with_delta else None
    h, y = residual_rmsnorm(xf, df, w, eps)
    torch.autograd.backward([h, y], [dh, dy])

    xu = x.clone().requires_grad_(True)
    du = d.clone().requires_grad_(True) if with_delta else None
    hu = xu + du if with_delta else xu
    yu = rmsnorm(hu, w, eps)
    torch.autograd.backward([hu, yu], [dh, dy])

    assert torch.equal(h, hu)
    assert torch.equal(y, yu)
    torch.testing.assert_close(xf.grad, xu.grad, rtol=8e-3, atol=8e-3)
    if with_delta:
        assert torch.equal(df.grad, xf.grad)

    # fp32 reference of the same function
    x32 = x.float().requires_grad_(True)
    h32 = x32 + d.float() if with_delta else x32
    hr = h32.to(torch.bfloat16).float()
    y32 = w.float() * (hr * torch.rsqrt(hr.pow(2).mean(-1, keepdim=True) + eps))
    torch.autograd.backward([h32, y32], [dh.float(), dy.float()])
    torch.testing.assert_close(xf.grad.float(), x32.grad, rtol=2e-2, atol=2e-2)


def _layer_and_inputs(dtype=torch.bfloat16):
    from transformers.models.qwen2 import modeling_qwen2 as m

    cfg = qlora_step.qwen2_config(hidden_size=256, intermediate_size=512, num_hidden_layers=1,
                                  num_attention_heads=2, num_key_value_heads=1, vocab_size=128)
    torch.manual_seed(0)
    with torch.device("cuda"):
        layer = m.Qwen2DecoderLayer(cfg, 0).to(dtype)
        rot = m.Qwen2RotaryEmbedding(cfg)
    layer.requires_grad_(False)
    with torch.no_grad():
        layer.input_layernorm.weight.normal_(1.0, 0.1)
        layer.post_attention_layernorm.weight.normal_(1.0, 0.1)
    x = torch.randn(2, 96, 256, device="cuda").to(dtype)
    pos = torch.arange(96, device="cuda")[None].expand(2, -1)
    cos, sin = rot(x, pos)
    return layer, x, (cos.to(dtype), sin.to(dtype)), pos


def test_patched_decoder_layer():
    from transformers.models.qwen2 import modeling_qwen2 as m

    hackathon_amd.apply()
    layer, x, pe, pos = _layer_and_inputs()
    dout = torch.randn_like(x)

    xa = x.clone().requires_grad_(True)
    out = layer(xa, position_embeddings=pe, position_ids=pos)
    out.backward(dout)
    xb = x.clone().requires_grad_(True)
    ref = m.Qwen2DecoderLayer.forward._original(layer, xb, position_embeddings=pe,
                                                position_ids=pos)
    ref.backward(dout)
    assert torch.equal(out, ref)
    torch.testing.assert_close(xa.grad, xb.grad, rtol=2e-2, atol=2e-2)

    # fp32 copy of the layer, transformers' own code (no patch)
    l32 = copy.deepcopy(layer).float()
    x32 = x.float().requires_grad_(True)
    qlora_step._unpatch_transformers()
    try:
        o32 = l32(x32, position_embeddings=(pe[0].float(), pe[1].float()), position_ids=pos)
        o32.backward(dout.float())
    finally:
        hackathon_amd.apply()
    torch.testing.assert_close(out.float(), o32, rtol=3e-2, atol=3e-2)
    err = (xa.grad.float() - x32.grad).norm() / x32.grad.norm()
    assert err < 2e-2, err
