"""Where a fused head loss plugs into training: Qwen2ForCausalLM.forward and a trainer's
compute_loss. Both fused variants (`fused_ce`, `cross_entropy`) hook these two places, as the
reference's do (solution/fused_ce.py:222-355, solution/cross_entropy.py:175-321); this module
holds the plumbing they share, and each variant supplies only its own rules and loss.

  - Eligibility is a table of named refusals, each a predicate over (trainer, model, inputs)
    or over the causal LM. A call is fused only when no refusal applies; otherwise the
    original code runs untouched. `refusal(...)` names the first one that applies.
  - The model hook replaces Qwen2ForCausalLM.forward by a dispatcher that asks the variant
    whether to take this call. A taken call runs the decoder body, hands its last hidden
    state to the variant's head loss and returns a CausalLMOutputWithPast without logits.
  - The trainer hook replaces compute_loss by a dispatcher that runs the variant's armed loss
    (the model hook fires inside it) and then logs TRL's metrics from the per-row statistics
    the kernels produced.
"""

from __future__ import annotations

import torch

from . import _common

STEP_ATTR = "_soup_chunked_step"  # where a rewind recorder finds the per-token loss of a step


# ---- eligibility -----------------------------------------------------------------------------
def refusal(checks, *args):
    """Name of the first check in `checks` ((name, predicate) pairs) whose predicate holds for
    `args`, or None when every check passes."""
    for name, applies in checks:
        if applies(*args):
            return name
    return None


def _args(trainer):
    return getattr(trainer, "args", None)


# Refusals both variants apply to a compute_loss call (trainer, model, inputs), in the terms of
# trl's SFTTrainer: a fused call must be plain NLL on labelled, masked inputs, with the trainer
# state TRL's metrics are logged into (solution/fused_ce.py:285-303,
# solution/cross_entropy.py:232-256).
TRAINER_REFUSALS = (
    ("trainer without args", lambda t, m, i: _args(t) is None),
    ("model is not a torch module", lambda t, m, i: not isinstance(m, torch.nn.Module)),
    ("inputs are not a dict", lambda t, m, i: not isinstance(i, dict)),
    ("liger kernel loss", lambda t, m, i: bool(getattr(_args(t), "use_liger_kernel", False))),
    ("loss type other than nll", lambda t, m, i: getattr(_args(t), "loss_type", "nll") != "nll"),
    ("custom compute_loss_func", lambda t, m, i: getattr(t, "compute_loss_func", None) is not None),
    ("label smoothing", lambda t, m, i: getattr(t, "label_smoother", None) is not None),
    ("virtual tokens", lambda t, m, i: bool(getattr(t, "num_virtual_tokens", 0))),
    ("auxiliary loss", lambda t, m, i: bool(getattr(t, "aux_loss_enabled", False))),
    ("trainer keeps no TRL metrics",
     lambda t, m, i: not (hasattr(t, "_metrics") and hasattr(t, "_total_train_tokens"))),
    ("no labels", lambda t, m, i: "labels" not in i),
    ("no attention mask", lambda t, m, i: "attention_mask" not in i),
    ("shift_labels given", lambda t, m, i: "shift_labels" in i),
)


def base_model(model):
    """The model under a peft wrapper (`get_base_model`), else the model itself."""
    get = getattr(model, "get_base_model", None)
    return get() if callable(get) else model


def is_qwen2_causal_lm(model):
    from transformers.models.qwen2.modeling_qwen2 import Qwen2ForCausalLM

    return isinstance(model, Qwen2ForCausalLM)


def head_refusal(lm, dtypes=None):
    """Why `lm`'s output head cannot take the fused path, or None: it must be a frozen,
    bias-free nn.Linear on the GPU (in one of `dtypes`, when given) with no logit
    soft-capping (solution/fused_ce.py:236-246, solution/cross_entropy.py:183-187)."""
    head = getattr(lm, "lm_head", None)
    weight = getattr(head, "weight", None)
    checks = (
        ("head is not a plain Linear", lambda: type(head) is not torch.nn.Linear),
        ("head has a bias", lambda: head.bias is not None),
        ("head weight is trained", lambda: weight.requires_grad),
        ("head weight is not on the GPU", lambda: not _common.on_gpu(weight)),
        ("head dtype not supported", lambda: dtypes is not None and weight.dtype not in dtypes),
        ("logit soft-capping",
         lambda: getattr(getattr(lm, "config", None), "final_logit_softcapping", None) is not None),
    )
    return refusal(checks)


# ---- the model hook --------------------------------------------------------------------------
def _chain(fn):
    """`fn` and the functions it wraps, outermost first (each hook keeps `_original`)."""
    while fn is not None:
        yield fn
        fn = getattr(fn, "_original", None)


def installed(fn, variant):
    """The dispatcher of `variant` in the chain of hooks ending at `fn`, or None."""
    return next((f for f in _chain(fn) if getattr(f, "_head_variant", None) == variant), None)


def install_model_hook(variant, wants, head_loss):
    """Put `variant`'s dispatcher in front of Qwen2ForCausalLM.forward, stacking on any forward
    already there; nothing happens when that variant's dispatcher is already in the chain.
    `wants(model, labels, logits_to_keep, kwargs)` decides per call; a taken call returns
    CausalLMOutputWithPast(loss=head_loss(model, hidden, labels, attention_mask, kwargs),
    logits=None, ...)."""
    from transformers.modeling_outputs import CausalLMOutputWithPast
    from transformers.models.qwen2 import modeling_qwen2

    wrapped = modeling_qwen2.Qwen2ForCausalLM.forward
    if installed(wrapped, variant) is not None:
        return

    def forward(self, input_ids=None, attention_mask=None, position_ids=None,
                past_key_values=None, inputs_embeds=None, labels=None, use_cache=None,
                logits_to_keep=0, **kwargs):
        call = dict(input_ids=input_ids, attention_mask=attention_mask,
                    position_ids=position_ids, past_key_values=past_key_values,
                    inputs_embeds=inputs_embeds, use_cache=use_cache)
        if not wants(self, labels, logits_to_keep, kwargs):
            return wrapped(self, labels=labels, logits_to_keep=logits_to_keep, **call, **kwargs)
        kwargs.pop("return_dict", None)  # the body returns a ModelOutput either way
        body = self.model(**call, **kwargs)
        loss = head_loss(self, body.last_hidden_state, labels, attention_mask, kwargs)
        return CausalLMOutputWithPast(loss=loss, logits=None,
                                      past_key_values=body.past_key_values,
                                      hidden_states=body.hidden_states,
                                      attentions=body.attentions)

    forward._original = wrapped
    forward._head_variant = variant
    forward._solution_patch = True
    modeling_qwen2.Qwen2ForCausalLM.forward = forward


def remove_model_hook(variant):
    """Restore the forward that `variant`'s dispatcher wrapped (dropping any hook stacked on
    top of it later)."""
    from transformers.models.qwen2 import modeling_qwen2

    hook = installed(modeling_qwen2.Qwen2ForCausalLM.forward, variant)
    if hook is not None:
        modeling_qwen2.Qwen2ForCausalLM.forward = hook._original


def plain_training_call(logits_to_keep, kwargs):
    """A forward that asks for every position's logits in a ModelOutput: the calls a fused
    head loss may answer without logits."""
    return (isinstance(logits_to_keep, int) and logits_to_keep == 0
            and kwargs.get("return_dict", True) is not False)


# ---- the trainer hook ------------------------------------------------------------------------
def install_trainer_hook(variant, trainer_cls, eligible, armed_loss, on_fallback=None):
    """Put `variant`'s dispatcher in front of `trainer_cls.compute_loss` (nothing happens when it
    is already in that method's chain). An eligible call
    (`eligible(trainer, model, inputs)`) drops the prediction-only flag, turns the KV cache off
    and returns the loss of `armed_loss(trainer, model, inputs, num_items_in_batch) ->
    (loss, outputs)`; any other call first runs `on_fallback(trainer)` (if given) and then the
    original compute_loss."""
    wrapped = trainer_cls.compute_loss
    if installed(wrapped, variant) is not None:
        return

    def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
        if not eligible(self, model, inputs):
            if on_fallback is not None:
                on_fallback(self)
            return wrapped(self, model, inputs, return_outputs=return_outputs,
                           num_items_in_batch=num_items_in_batch)
        inputs.pop("_prediction_loss_only", None)
        inputs["use_cache"] = False
        loss, outputs = armed_loss(self, model, inputs, num_items_in_batch)
        return (loss, outputs) if return_outputs else loss

    compute_loss._original = wrapped
    compute_loss._head_variant = variant
    compute_loss._solution_patch = True
    trainer_cls.compute_loss = compute_loss


def remove_trainer_hook(variant, trainer_cls):
    """Restore the compute_loss that `variant`'s dispatcher wrapped on `trainer_cls`."""
    hook = installed(trainer_cls.__dict__.get("compute_loss"), variant)
    if hook is not None:
        trainer_cls.compute_loss = hook._original


def default_trainer_class():
    """trl's SFTTrainer when trl is importable, else None."""
    try:
        from trl import SFTTrainer
    except ImportError:
        return None
    return SFTTrainer


def log_trl_metrics(trainer, mode, attention_mask, entropy, correct, labelled, count_tokens):
    """Append entropy, num_tokens and mean_token_accuracy to trainer._metrics[mode] the way
    trl 0.29.1's SFTTrainer.compute_loss computes them: `entropy` is this process's masked mean
    entropy (a tensor), averaged over processes; `correct` / `labelled` are this process's
    counts of correct and labelled tokens, summed over processes; the token count grows by the
    attention mask's sum when `count_tokens`."""
    gather = trainer.accelerator.gather_for_metrics
    with torch.no_grad():
        trainer._metrics[mode]["entropy"].append(gather(entropy).mean().item())
        if count_tokens:
            trainer._total_train_tokens += gather(attention_mask.sum()).sum().item()
        trainer._metrics[mode]["num_tokens"] = [trainer._total_train_tokens]
        hits, seen = gather(correct).sum(), gather(labelled).sum()
        accuracy = (hits / seen).item() if seen > 0 else 0.0
    trainer._metrics[mode]["mean_token_accuracy"].append(accuracy)


def entropy_from_logits(logits, chunk_size=128):
    """Per-position entropy of softmax(logits), -sum(p log p) with log p = log_softmax, in
    chunks of rows: the formula of trl's `trl.trainer.utils.entropy_from_logits` (trl 0.29.1,
    not installed here)."""
    flat = logits.reshape(-1, logits.shape[-1])
    out = torch.empty(flat.shape[0], dtype=flat.dtype, device=flat.device)
    for start in range(0, flat.shape[0], chunk_size):
        logp = torch.nn.functional.log_softmax(flat[start:start + chunk_size], dim=-1)
        out[start:start + chunk_size] = -(logp.exp() * logp).sum(-1)
    return out.reshape(logits.shape[:-1])
