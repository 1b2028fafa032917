"""The QLoRA training step the kernel set serves: a Qwen2.5-shaped causal LM with NF4 bases
and LoRA adapters on every projection, one forward + backward + AdamW step on the adapters.

The reference runs this step inside an external trainer (soup-cli -> TRL SFTTrainer ->
transformers Qwen2ForCausalLM -> peft LoRA on bitsandbytes 4-bit; solution/__init__.py:1-15)
and installs its kernels with `apply()`. None of that trainer stack is available here, so
this module builds the same model shape from a local `Qwen2Config` with random weights
(no checkpoint, no network), swaps every q/k/v/o/gate/up/down projection for
`LoraLinear4bit(Linear4bit)` and runs the step either
  - patched: `hackathon_amd.apply()` installed and the fused head loss armed, so every
    RMSNorm (with the decoder layer's residual adds), RoPE, attention, SwiGLU, NF4 linear,
    LoRA cast/GEMM/add, the lm_head + CE and the AdamW update run on the gfx950 kernels; or
  - eager: the plain PyTorch-ROCm path (torch-op dequant, hipBLASLt GEMMs through F.linear,
    transformers' own RMSNorm/RoPE/MLP, torch SDPA, full-logits ForCausalLMLoss and torch's
    foreach AdamW), the baseline.
"""

from __future__ import annotations

import contextlib
import types

import torch

from . import cross_entropy, eager, lora, quant

QWEN25_7B = dict(hidden_size=3584, intermediate_size=18944, num_hidden_layers=28,
                 num_attention_heads=28, num_key_value_heads=4, vocab_size=152064,
                 rms_norm_eps=1e-6, rope_theta=1e6, max_position_embeddings=32768,
                 tie_word_embeddings=False, hidden_act="silu")

PROJECTIONS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
               "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def qwen2_config(**overrides):
    from transformers import Qwen2Config

    kw = dict(QWEN25_7B)
    kw.update(overrides)
    cfg = Qwen2Config(**kw)
    cfg._attn_implementation = "sdpa"
    return cfg


def build_qlora_model(config, device="cuda", r=16, alpha=32, dropout=0.0, seed=0,
                      a_std=0.25, b_std=0.01, compute_dtype=torch.bfloat16,
                      blocksize=64):
    """Random-init Qwen2ForCausalLM in bf16 on `device`, all projections NF4 (double-quantised
    absmax, blocksize 64) + LoRA (r, alpha) with A ~ N(0, a_std^2), B ~ N(0, b_std^2) in fp32.
    Only the adapters require grad."""
    from transformers.models.qwen2.modeling_qwen2 import Qwen2ForCausalLM

    torch.manual_seed(seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(compute_dtype)
    try:
        with torch.device(device):
            model = Qwen2ForCausalLM(config)
    finally:
        torch.set_default_dtype(prev)
    model.requires_grad_(False)
    gen = torch.Generator(device=device).manual_seed(seed + 1)
    for layer in model.model.layers:
        for path in PROJECTIONS:
            owner_name, child = path.split(".")
            owner = getattr(layer, owner_name)
            lin = getattr(owner, child)
            base = quant.Linear4bit.from_weight(lin.weight.data, bias=lin.bias,
                                                compute_dtype=compute_dtype, blocksize=blocksize)
            ll = lora.LoraLinear4bit(base, r=r, lora_alpha=alpha, lora_dropout=dropout,
                                     compute_dtype=compute_dtype)
            with torch.no_grad():
                ll.lora_A["default"].weight.normal_(0.0, a_std, generator=gen)
                ll.lora_B["default"].weight.normal_(0.0, b_std, generator=gen)
            setattr(owner, child, ll)
            del lin
    model.train()
    return model


def lora_parameters(model):
    return [p for p in model.parameters() if p.requires_grad]


def make_batch(batch, seq, vocab, device="cuda", seed=0):
    """Uniform random token ids; labels = ids (the causal shift happens in the loss)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    ids = torch.randint(0, vocab, (batch, seq), generator=g).to(device)
    return ids, ids.clone()


def _unpatch_transformers():
    """Restore transformers' originals of every class attribute `apply()` patched."""
    from transformers.models.qwen2 import modeling_qwen2 as m

    for owner, name in ((m.Qwen2RMSNorm, "forward"), (m.Qwen2MLP, "forward"),
                        (m.Qwen2ForCausalLM, "forward"), (m, "apply_rotary_pos_emb"),
                        (m.Qwen2DecoderLayer, "forward"), (m.Qwen2Attention, "forward")):
        fn = getattr(owner, name)
        while getattr(fn, "_original", None) is not None:  # patches may stack
            fn = fn._original
        setattr(owner, name, fn)
    from transformers.modeling_utils import AttentionInterface

    orig = getattr(AttentionInterface._global_mapping["sdpa"], "_original", None)
    if orig is not None:
        AttentionInterface._global_mapping["sdpa"] = orig
    import hackathon_amd

    hackathon_amd._applied.clear()


@contextlib.contextmanager
def eager_mode(model):
    """Run `model` on the plain PyTorch path (the baseline) inside the block."""
    _unpatch_transformers()
    saved = []
    for mod in model.modules():
        if isinstance(mod, lora.LoraLinear4bit):
            saved.append(mod)
            mod.forward = types.MethodType(eager.lora_forward_eager, mod)
        elif isinstance(mod, quant.Linear4bit):
            saved.append(mod)
            mod.forward = types.MethodType(eager.linear4bit_eager, mod)
    try:
        yield model
    finally:
        for mod in saved:
            del mod.forward


def patched_mode():
    """Install every kernel patch (idempotent)."""
    import hackathon_amd

    hackathon_amd.apply()


class QLoRAStep:
    """forward + backward + AdamW on the adapters. `fused_head` arms the chunked lm_head + CE
    for the forward (what the reference's trainer hook does, solution/cross_entropy.py:294);
    `fused_adamw` updates the adapters with `optim.FusedAdamW` (one HIP launch) instead of
    torch's foreach AdamW."""

    def __init__(self, model, lr=1e-4, fused_head=True, fused_adamw=None):
        self.model = model
        self.fused_head = fused_head
        if fused_adamw is None:
            fused_adamw = fused_head
        params = lora_parameters(model)
        if fused_adamw:
            from .optim import FusedAdamW

            self.opt = FusedAdamW(params, lr=lr, betas=(0.9, 0.999), weight_decay=0.0)
        else:
            self.opt = torch.optim.AdamW(params, lr=lr, betas=(0.9, 0.999), weight_decay=0.0,
                                         foreach=True)

    def forward_backward(self, input_ids, labels):
        if self.fused_head:
            cross_entropy.STATE.armed = True
        try:
            out = self.model(input_ids=input_ids, labels=labels, use_cache=False)
        finally:
            cross_entropy.STATE.armed = False
        out.loss.backward()
        return out.loss.detach()

    def __call__(self, input_ids, labels):
        loss = self.forward_backward(input_ids, labels)
        self.opt.step()
        self.opt.zero_grad(set_to_none=True)
        return loss
