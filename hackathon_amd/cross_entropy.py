"""Fused, chunked lm_head + cross-entropy + entropy + argmax over the vocabulary
(drop-in for solution/cross_entropy.py, the variant `apply()` installs).

The full logits never exist. Rows go through in chunks of CHUNK_ROWS tokens
(solution/cross_entropy.py:11-21):
  1. logits_chunk = hidden_chunk @ W.T                 qlora_gemm, in the matmul dtype
  2. one workgroup per row, two sweeps over the vocab:  qlora_ce_rows (ignore_mode 1)
       sweep 1: online max / log-sum-exp, sum(p*z) for the entropy, first argmax, z[label]
       sweep 2: dz = (softmax - onehot) * GRAD_GAIN / denominator, IN PLACE over the chunk
  3. grad_h_chunk = dz @ W                               qlora_gemm_ws, fp32 output, against
                                                         the cached W^T (k = vocabulary
                                                         contiguous), split over K
The hidden gradient is taken in forward (the head is frozen); backward only rescales it.
"""

from __future__ import annotations

import torch

from . import _common, _lib
from . import gemm as _gemm

IGNORE_INDEX = -100
CHUNK_ROWS = 512
BLOCK_V = 4096  # the reference's vocab block (solution/cross_entropy.py:39); tiles are internal
# dz is stored in the 16-bit matmul dtype before dz @ W; it is stored multiplied by GRAD_GAIN
# (a power of two, exact) so (p - onehot)/num_tokens does not underflow fp16, and divided back
# in fp32 (solution/cross_entropy.py:40-44).
GRAD_GAIN = 65536.0
STEP_ATTR = "_soup_chunked_step"


def ce_chunk(logits, target, token_loss, entropy, pred, grad_scale, write_grad):
    """Run the row kernel on one logits chunk (solution/cross_entropy.py:48-90 semantics)."""
    n, vocab = logits.shape
    if n == 0:
        return
    _lib.call("qlora_ce_rows", logits.data_ptr(), _lib.tag(logits.dtype), logits.stride(0), n,
              vocab, target.data_ptr(), token_loss.data_ptr(), entropy.data_ptr(), None,
              pred.data_ptr(), 1, int(bool(write_grad)), float(grad_scale),
              _lib.stream_of(logits))


class FusedLinearCrossEntropy(torch.autograd.Function):
    """loss = sum_rows CE(hidden @ W.T, target) / denominator, plus per-token loss, entropy and
    argmax, without the full logits (solution/cross_entropy.py:93-138)."""

    @staticmethod
    def forward(ctx, hidden, weight, target, denominator, matmul_dtype, chunk_rows):
        _lib.require_device(hidden, weight)
        shape = hidden.shape
        h2 = hidden.reshape(-1, shape[-1])
        tgt = target.reshape(-1).to(device=hidden.device, dtype=torch.int64).contiguous()
        n_rows, vocab = h2.shape[0], weight.shape[0]
        dev = hidden.device
        with_grad = ctx.needs_input_grad[0]
        denom = float(denominator)
        grad_scale = GRAD_GAIN / denom if denom else 0.0

        token_loss = torch.empty(n_rows, dtype=torch.float32, device=dev)
        entropy = torch.empty(n_rows, dtype=torch.float32, device=dev)
        pred = torch.empty(n_rows, dtype=torch.int64, device=dev)
        grad_h = torch.empty((n_rows, shape[-1]), dtype=torch.float32, device=dev) \
            if with_grad else None
        mm16 = matmul_dtype in (torch.float16, torch.bfloat16)
        with torch.autocast(device_type=dev.type, enabled=False):
            w = weight.to(matmul_dtype).contiguous()
            buf = _gemm.padded_rows(min(chunk_rows, max(n_rows, 1)), vocab, matmul_dtype, dev)
            for start in range(0, n_rows, chunk_rows):
                stop = min(start + chunk_rows, n_rows)
                hc = h2[start:stop].to(matmul_dtype)
                logits = buf[: stop - start]
                if mm16:
                    _gemm.gemm(hc, w, out=logits)
                else:
                    torch.mm(hc, w.t(), out=logits)
                ce_chunk(logits, tgt[start:stop], token_loss[start:stop], entropy[start:stop],
                         pred[start:stop], grad_scale, with_grad)
                if with_grad:
                    if mm16:
                        _gemm.gemm(logits, _gemm.transposed_frozen(w), out=grad_h[start:stop])
                    else:
                        grad_h[start:stop] = logits @ w
            del w, buf
        loss = token_loss.sum() / denominator
        ctx.save_for_backward(grad_h)
        ctx.shape, ctx.dtype = shape, hidden.dtype
        ctx.mark_non_differentiable(token_loss, entropy, pred)
        return loss, token_loss.view(shape[:-1]), entropy.view(shape[:-1]), pred.view(shape[:-1])

    @staticmethod
    def backward(ctx, grad_loss, _grad_token_loss, _grad_entropy, _grad_pred):
        (grad_h,) = ctx.saved_tensors
        if grad_h is None:
            return None, None, None, None, None, None
        grad = grad_h * (grad_loss.float() / GRAD_GAIN)
        return grad.view(ctx.shape).to(ctx.dtype), None, None, None, None, None


class ChunkedStep:
    """What the fused forward leaves for the metrics (solution/cross_entropy.py:141-150)."""

    def __init__(self, token_entropy, token_loss, pred, target):
        self.token_entropy = token_entropy
        self.token_loss = token_loss
        labelled = target != IGNORE_INDEX
        self.labelled = labelled.sum()
        self.correct = ((pred == target) & labelled).sum()


def shift_labels_of(labels):
    """labels moved one left, as ForCausalLMLoss does (solution/cross_entropy.py:153-155)."""
    return torch.nn.functional.pad(labels, (0, 1), value=IGNORE_INDEX)[..., 1:]


def fused_causal_lm_loss(hidden, weight, labels, num_items_in_batch=None, shift_labels=None,
                         chunk_rows=CHUNK_ROWS):
    """ForCausalLMLoss(hidden @ weight.T, labels) and a ChunkedStep, without the full logits
    (solution/cross_entropy.py:158-172)."""
    target = shift_labels if shift_labels is not None else shift_labels_of(labels)
    target = target.to(hidden.device)
    if num_items_in_batch is None:
        denominator = (target != IGNORE_INDEX).sum()
    elif torch.is_tensor(num_items_in_batch):
        denominator = num_items_in_batch.to(hidden.device)
    else:
        denominator = num_items_in_batch
    matmul_dtype = _common.autocast_dtype() or torch.promote_types(hidden.dtype, weight.dtype)
    loss, token_loss, entropy, pred = FusedLinearCrossEntropy.apply(
        hidden, weight, target, denominator, matmul_dtype, chunk_rows)
    return loss, ChunkedStep(entropy, token_loss, pred, target)


class _State:
    armed = False
    step = None


STATE = _State()


def _head_ok(lm):
    head = getattr(lm, "lm_head", None)
    return (type(head) is torch.nn.Linear and head.bias is None
            and not head.weight.requires_grad and _common.on_gpu(head.weight)
            and getattr(lm.config, "final_logit_softcapping", None) is None)


def _patch_causal_lm():
    """Qwen2ForCausalLM.forward computes the fused loss when armed by a trainer hook, else the
    original (solution/cross_entropy.py:190-222)."""
    from transformers.modeling_outputs import CausalLMOutputWithPast
    from transformers.models.qwen2 import modeling_qwen2 as m

    original = m.Qwen2ForCausalLM.forward
    if getattr(original, "_solution_patch", False):
        return

    def forward(self, input_ids=None, attention_mask=None, position_ids=None,
                past_key_values=None, inputs_embeds=None, labels=None, use_cache=None,
                logits_to_keep=0, **kwargs):
        if not (STATE.armed and labels is not None and _common.on_gpu(labels)
                and isinstance(logits_to_keep, int) and logits_to_keep == 0
                and kwargs.get("return_dict", True) is not False and _head_ok(self)):
            return original(self, input_ids=input_ids, attention_mask=attention_mask,
                            position_ids=position_ids, past_key_values=past_key_values,
                            inputs_embeds=inputs_embeds, labels=labels, use_cache=use_cache,
                            logits_to_keep=logits_to_keep, **kwargs)
        STATE.armed = False
        outputs = self.model(input_ids=input_ids, attention_mask=attention_mask,
                             position_ids=position_ids, past_key_values=past_key_values,
                             inputs_embeds=inputs_embeds, use_cache=use_cache, **kwargs)
        loss, STATE.step = fused_causal_lm_loss(
            outputs.last_hidden_state, self.lm_head.weight, labels,
            num_items_in_batch=kwargs.get("num_items_in_batch"),
            shift_labels=kwargs.get("shift_labels"))
        return CausalLMOutputWithPast(loss=loss, logits=None,
                                      past_key_values=outputs.past_key_values,
                                      hidden_states=outputs.hidden_states,
                                      attentions=outputs.attentions)

    forward._solution_patch = True
    forward._original = original
    m.Qwen2ForCausalLM.forward = forward


def _causal_lm_of(trainer, model):
    """The Qwen2ForCausalLM under accelerate / peft wrappers (solution/cross_entropy.py:225-229)."""
    unwrap = getattr(getattr(trainer, "accelerator", None), "unwrap_model", None)
    inner = unwrap(model) if callable(unwrap) else model
    get_base = getattr(inner, "get_base_model", None)
    return get_base() if callable(get_base) else inner


def _can_fuse(trainer, model, inputs):
    """Whether this compute_loss call may take the fused head: a training step of plain NLL on
    a Qwen2 causal LM whose frozen head lives on the GPU, with the trainer state TRL's metrics
    need and no other loss machinery (solution/cross_entropy.py:232-262)."""
    from transformers.models.qwen2.modeling_qwen2 import Qwen2ForCausalLM

    args = getattr(trainer, "args", None)
    if not (isinstance(model, torch.nn.Module) and isinstance(inputs, dict) and args is not None):
        return False
    if not getattr(trainer.model, "training", False):
        return False
    if "labels" not in inputs or "shift_labels" in inputs or "attention_mask" not in inputs:
        return False
    if not _common.on_gpu(inputs["labels"], inputs["attention_mask"]):
        return False
    if getattr(args, "use_liger_kernel", False) or getattr(args, "loss_type", "nll") != "nll":
        return False
    if getattr(trainer, "num_virtual_tokens", 0) or getattr(trainer, "aux_loss_enabled", False):
        return False
    if getattr(trainer, "compute_loss_func", None) is not None or \
            getattr(trainer, "label_smoother", None) is not None:
        return False
    if getattr(trainer, "_soup_chunked_head_loss", None) is not None:
        return False
    if not all(hasattr(trainer, name) for name in ("_metrics", "_total_train_tokens")):
        return False
    lm = _causal_lm_of(trainer, model)
    return isinstance(lm, Qwen2ForCausalLM) and _head_ok(lm)


def entropy_from_logits(logits, chunk_size=128):
    """Per-position entropy of softmax(logits), by the formula of trl's
    `trl.trainer.utils.entropy_from_logits` (trl 0.29.1, not installed here): -sum(p log p)
    with log p = log_softmax, in chunks of rows."""
    flat = logits.reshape(-1, logits.shape[-1])
    parts = []
    for chunk in flat.split(chunk_size, dim=0):
        logp = torch.nn.functional.log_softmax(chunk, dim=-1)
        parts.append(-(torch.exp(logp) * logp).sum(-1))
    return torch.cat(parts, dim=0).reshape(logits.shape[:-1])


def _log_metrics(trainer, mode, inputs, step):
    """entropy, num_tokens and mean_token_accuracy as trl 0.29.1 SFTTrainer.compute_loss logs
    them (attention_mask present, no virtual tokens), from the fused step's per-row statistics
    instead of the logits (solution/cross_entropy.py:265-287)."""
    gather = trainer.accelerator.gather_for_metrics
    attention_mask = inputs["attention_mask"]
    with torch.no_grad():
        entropy = torch.sum(step.token_entropy * attention_mask) / attention_mask.sum()
        entropy = gather(entropy).mean().item()
    trainer._metrics[mode]["entropy"].append(entropy)
    if mode == "train":
        trainer._total_train_tokens += gather(attention_mask.sum()).sum().item()
    trainer._metrics[mode]["num_tokens"] = [trainer._total_train_tokens]
    with torch.no_grad():
        correct = gather(step.correct)
        total = gather(step.labelled)
        total_sum = total.sum()
        accuracy = (correct.sum() / total_sum).item() if total_sum > 0 else 0.0
    trainer._metrics[mode]["mean_token_accuracy"].append(accuracy)


def _patch_trainer(trainer_cls=None):
    """Arm the fused head inside `trainer_cls.compute_loss` (default: trl's SFTTrainer; returns
    False when trl is not importable) and log TRL's metrics from the fused statistics
    (solution/cross_entropy.py:290-316). The loss itself comes from the parent class's
    compute_loss (transformers' Trainer), which calls the model with the labels."""
    if trainer_cls is None:
        try:
            from trl import SFTTrainer as trainer_cls
        except ImportError:
            return False
    original = trainer_cls.compute_loss
    if getattr(original, "_solution_patch", False):
        return True

    def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
        if not _can_fuse(self, model, inputs):
            return original(self, model, inputs, return_outputs=return_outputs,
                            num_items_in_batch=num_items_in_batch)
        mode = "train" if self.model.training else "eval"
        inputs.pop("_prediction_loss_only", None)
        labels = inputs["labels"]
        inputs["use_cache"] = False
        STATE.armed, STATE.step = True, None
        try:
            loss, outputs = super(trainer_cls, self).compute_loss(
                model, inputs, return_outputs=True, num_items_in_batch=num_items_in_batch)
        finally:
            STATE.armed = False
        step, STATE.step = STATE.step, None
        if step is None:
            # the model took its original path after all (it has logits): same metrics from them
            with torch.no_grad():
                logits = outputs.logits
                step = ChunkedStep(entropy_from_logits(logits), None, logits.argmax(dim=-1),
                                   shift_labels_of(labels))
            setattr(self, STEP_ATTR, None)
        else:
            setattr(self, STEP_ATTR, step)
        _log_metrics(self, mode, inputs, step)
        return (loss, outputs) if return_outputs else loss

    compute_loss._solution_patch = True
    compute_loss._original = original
    trainer_cls.compute_loss = compute_loss
    return True


def patch(trainer_cls=None):
    """Install the model hook and the trainer hook that arms it (solution/cross_entropy.py:
    319-321). The trainer hook goes on `trainer_cls`, by default trl's SFTTrainer when trl is
    importable (it is not in this image, so only the model hook is installed then)."""
    _patch_causal_lm()
    _patch_trainer(trainer_cls)
