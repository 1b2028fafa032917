"""The trainer hooks on the GPU: a real (small, random) Qwen2ForCausalLM trained through the
stub SFTTrainer. The fused path (hook armed, no logits) and the trainer's own logits path give
the same loss (rtol 2e-3: fp16/bf16 head GEMM in 512-row chunks vs one bf16 GEMM), the same
TRL metrics (entropy rtol 2e-3, accuracy within one token in 1e3, num_tokens exact) and the
same adapter-free hidden gradient direction; the per-token loss is left for a recorder."""

import pytest
import torch

import hackathon_amd
from hackathon_amd import cross_entropy, fused_ce, qlora_step

from _trainer_stub import make_trainer, new_sft_class

pytestmark = pytest.mark.gpu


def _model(dtype):
    from transformers.models.qwen2.modeling_qwen2 import Qwen2ForCausalLM

    cfg = qlora_step.qwen2_config(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                  num_attention_heads=2, num_key_value_heads=1, vocab_size=1024)
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        with torch.device("cuda"):
            model = Qwen2ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    model.requires_grad_(False)
    model.model.embed_tokens.weight.requires_grad_(True)  # something to train
    model.train()
    return model


def _inputs(seed=1):
    g = torch.Generator(device="cpu").manual_seed(seed)
    ids = torch.randint(0, 1024, (2, 160), generator=g).cuda()
    labels = ids.clone()
    labels[:, :40] = -100   # prompt
    return {"input_ids": ids, "labels": labels,
            "attention_mask": torch.ones_like(ids)}


def _run(trainer, model):
    model.zero_grad(set_to_none=True)
    loss = trainer.compute_loss(model, _inputs())
    loss.backward()
    return float(loss.detach()), model.model.embed_tokens.weight.grad.float().clone()


def _compare(t_ref, t_fused, ref, fused):
    loss_r, grad_r = ref
    loss_f, grad_f = fused
    assert loss_f == pytest.approx(loss_r, rel=2e-3)
    m_r, m_f = t_ref._metrics["train"], t_fused._metrics["train"]
    assert m_f["entropy"][-1] == pytest.approx(m_r["entropy"][-1], rel=2e-3)
    assert m_f["num_tokens"] == m_r["num_tokens"]
    assert abs(m_f["mean_token_accuracy"][-1] - m_r["mean_token_accuracy"][-1]) <= 1e-3
    cos = torch.nn.functional.cosine_similarity(grad_f.flatten(), grad_r.flatten(), dim=0)
    assert cos > 0.999, float(cos)


def test_cross_entropy_trainer_hook():
    hackathon_amd.apply()
    Hooked = new_sft_class()
    model = _model(torch.bfloat16)
    ref_t = make_trainer(model, Hooked)
    ref = _run(ref_t, model)
    assert cross_entropy._patch_trainer(Hooked)
    t = make_trainer(model, Hooked)
    fused = _run(t, model)
    _compare(ref_t, t, ref, fused)
    step = getattr(t, cross_entropy.STEP_ATTR)
    assert step is not None and step.token_loss.shape == (2, 160)


def test_fused_ce_trainer_hook():
    hackathon_amd.apply()
    Hooked = new_sft_class()
    model = _model(torch.float16)
    ref_t = make_trainer(model, Hooked)
    ref = _run(ref_t, model)
    fused_ce.patch_qwen2_causal_lm()
    assert fused_ce.patch_sft_trainer(Hooked)
    try:
        t = make_trainer(model, Hooked)
        fused = _run(t, model)
    finally:
        fused_ce.unpatch()
    _compare(ref_t, t, ref, fused)
    assert getattr(t, fused_ce.STEP_ATTR).token_loss.shape == (2, 160)
