"""Adapter packing in one launch per model forward (adapter_packs, qlora_lora_pack_jobs).

Bar: bit-identical to packing each group on its own (qlora_lora_pack_group), and a model's
loss and adapter gradients bit-identical with and without the batched packing, also when the
adapters change between forwards without any version bump (writes through .data) and when a
backward runs after a later forward.
"""

import pytest
import torch

from hackathon_amd import adapter_packs, qlora_step
from hackathon_amd import gemm as _gemm

pytestmark = pytest.mark.gpu


def _factors(g, G, K, ns, scales):
    return [(torch.randn(16, K, device="cuda", generator=g) * 0.1,
             torch.randn(n, 16, device="cuda", generator=g) * 0.1, s)
            for n, s in zip(ns[:G], scales[:G])]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pack_jobs_equal_per_group_packs(dtype):
    print(f"pack jobs {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(3)
    groups = {}
    cases = [(3, 3584, (3584, 512, 512)), (1, 3584, (3584,)), (2, 3584, (18944, 18944)),
             (1, 18944, (3584,)), (4, 520, (24, 40, 8, 16)), (1, 8, (1,))]
    for i, (G, K, ns) in enumerate(cases):
        groups[i] = (_factors(g, G, K, ns, (2.0, 0.5, 1.25, 3.0)), dtype, 64)
    packs = adapter_packs._pack_all(groups, torch.device("cuda"))
    for i, (factors, _, pad) in groups.items():
        want = _gemm.lora_pack_group(factors, dtype, pad)
        got = packs[i]
        for w, t in zip(want, got):
            assert w.shape == t.shape and w.dtype == t.dtype
            assert torch.equal(w, t), f"case {cases[i]}"


def _tiny_model():
    cfg = qlora_step.qwen2_config(hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                                  num_attention_heads=4, num_key_value_heads=2, vocab_size=1000)
    model = qlora_step.build_qlora_model(cfg, "cuda", seed=0)
    ids, labels = qlora_step.make_batch(2, 64, cfg.vocab_size)
    return model, ids, labels


def _loss_and_grads(model, ids, labels):
    model.zero_grad(set_to_none=True)
    loss = qlora_step.QLoRAStep(model).forward_backward(ids, labels)
    return loss, [p.grad.clone() for p in qlora_step.lora_parameters(model)]


def _without_batching(monkeypatch):
    monkeypatch.setattr(adapter_packs, "pack_group", _gemm.lora_pack_group)


def test_batched_packs_give_the_same_step(monkeypatch):
    print("batched packs: step", flush=True)
    qlora_step.patched_mode()
    model, ids, labels = _tiny_model()
    calls = []
    real = adapter_packs._launch
    monkeypatch.setattr(adapter_packs, "_launch",
                        lambda plan: calls.append(plan.njobs) or real(plan))
    _loss_and_grads(model, ids, labels)               # registers the groups
    # change every adapter without a version bump: the next forward must see the new values
    with torch.no_grad():
        for p in qlora_step.lora_parameters(model):
            p.data.mul_(1.5).add_(0.01)
    loss_b, grads_b = _loss_and_grads(model, ids, labels)
    assert calls and calls[-1] == 4 * 2               # q/k/v, o, gate/up, down per layer
    with monkeypatch.context() as m:
        _without_batching(m)
        loss_r, grads_r = _loss_and_grads(model, ids, labels)
    assert torch.equal(loss_b, loss_r)
    for a, b in zip(grads_b, grads_r):
        assert torch.equal(a, b)


def test_backward_after_a_later_forward_reads_its_own_packs():
    print("batched packs: backward after a later forward", flush=True)
    qlora_step.patched_mode()
    model, ids, labels = _tiny_model()
    params = qlora_step.lora_parameters(model)
    _loss_and_grads(model, ids, labels)               # registers the groups
    want_loss, want = _loss_and_grads(model, ids, labels)
    model.zero_grad(set_to_none=True)
    from hackathon_amd import cross_entropy
    cross_entropy.STATE.armed = True
    try:
        out1 = model(input_ids=ids, labels=labels, use_cache=False)
    finally:
        cross_entropy.STATE.armed = False
    saved = [p.detach().clone() for p in params]
    with torch.no_grad():
        for p in params:
            p.data.mul_(-2.0)
    cross_entropy.STATE.armed = True
    try:
        model(input_ids=ids, labels=labels, use_cache=False)   # packs the changed adapters
    finally:
        cross_entropy.STATE.armed = False
    with torch.no_grad():
        for p, s in zip(params, saved):
            p.data.copy_(s)
    out1.loss.backward()
    assert torch.equal(out1.loss.detach(), want_loss)
    for p, w in zip(params, want):
        assert torch.equal(p.grad, w)
