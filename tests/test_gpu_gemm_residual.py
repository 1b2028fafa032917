"""The decoder layer's last add taken into the down projection's GEMM
(qlora_gemm_nt_cat_residual, fused_proj.LoraMLP with a residual).

Bar: bit-identical to the GEMM followed by torch's `residual + out` on every epilogue the GEMM
has (the LDS-staged tile store, the direct store for a row length that is not a multiple of
8, the split-K reduce), and a model's loss and adapter gradients bit-identical with and
without the fusion.
"""

import pytest
import torch

from hackathon_amd import gemm, lora, qlora_step, residual

pytestmark = pytest.mark.gpu

CASES = [
    # M, N, K, K2, dtype, ldc, ld_residual
    (4096, 3584, 18944, 64, torch.bfloat16, 3584, 3584),   # the 7B down projection
    (64, 3584, 2048, 64, torch.bfloat16, 3584, 3584),      # few rows: split-K
    (300, 1000, 640, 0, torch.float16, 1000, 1000),        # ragged tiles, no second segment
    (300, 1004, 640, 64, torch.bfloat16, 1008, 1016),      # a partial 8-column chunk
    (130, 1004, 128, 0, torch.bfloat16, 1004, 1008),       # unaligned output rows: direct store
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}x{c[1]}x{c[2]}+{c[3]}" for c in CASES])
def test_residual_gemm_equals_gemm_then_add(case):
    M, N, K, K2, dt, ldc, ldr = case
    print(f"residual gemm {case}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    a = torch.randn(M, K, device="cuda", generator=g).to(dt)
    b = (torch.randn(N, K, device="cuda", generator=g) * K ** -0.5).to(dt)
    a2 = b2 = None
    if K2:
        a2 = torch.randn(M, K2, device="cuda", generator=g).to(dt)
        b2 = (torch.randn(N, K2, device="cuda", generator=g) * 0.1).to(dt)
    r = torch.randn(M, ldr, device="cuda", generator=g).to(dt)[:, :N]
    want = torch.empty(M, ldc, device="cuda", dtype=dt)[:, :N]
    gemm.gemm_nt_cat(a, b, a2, b2, want)
    want = r + want
    got = torch.full((M, ldc), float("nan"), device="cuda", dtype=dt)[:, :N]
    gemm.gemm_nt_cat(a, b, a2, b2, got, residual=r)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def _model(dropout=0.0):
    cfg = qlora_step.qwen2_config(hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                                  num_attention_heads=4, num_key_value_heads=2, vocab_size=1000)
    model = qlora_step.build_qlora_model(cfg, "cuda", seed=0, dropout=dropout)
    ids, labels = qlora_step.make_batch(2, 64, cfg.vocab_size)
    return model, ids, labels


def _loss_and_grads(model, ids, labels):
    torch.manual_seed(5)
    lora._Seeds.gen = None   # the same dropout seeds on every call
    model.zero_grad(set_to_none=True)
    loss = qlora_step.QLoRAStep(model).forward_backward(ids, labels)
    return loss, [p.grad.clone() for p in qlora_step.lora_parameters(model)]


@pytest.mark.parametrize("p", [0.0, 0.05])
def test_step_equal_with_and_without_the_fused_add(monkeypatch, p):
    print(f"fused residual add: step, dropout {p}", flush=True)
    qlora_step.patched_mode()
    model, ids, labels = _model(p)
    used = []
    real = residual._mlp_with_residual
    monkeypatch.setattr(residual, "_mlp_with_residual",
                        lambda *a: used.append(real(*a)) or used[-1])
    loss_f, grads_f = _loss_and_grads(model, ids, labels)
    assert len(used) == 2 and all(u is not None for u in used)   # both layers fused the add
    with monkeypatch.context() as m:
        m.setattr(residual, "_mlp_with_residual", lambda *a: None)
        loss_r, grads_r = _loss_and_grads(model, ids, labels)
    assert torch.equal(loss_f, loss_r)
    for a, b in zip(grads_f, grads_r):
        assert torch.equal(a, b)


def test_hooked_mlp_keeps_the_plain_add():
    print("fused residual add: hooks", flush=True)
    qlora_step.patched_mode()
    model, ids, labels = _model()
    mlp = model.model.layers[0].mlp
    assert residual._plain_call(mlp)
    seen = []
    h = mlp.register_forward_hook(lambda mod, inp, out: seen.append(out.shape))
    try:
        assert not residual._plain_call(mlp)
        _loss_and_grads(model, ids, labels)
    finally:
        h.remove()
    assert seen == [(2, 64, 512)]
