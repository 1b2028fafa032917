"""Fused lm_head + cross-entropy + entropy + argmax over the vocabulary without the full
logits: drop-in for solution/cross_entropy.py, the variant `apply()` installs.

`fused_causal_lm_loss` is transformers' ForCausalLMLoss(hidden @ W.T, labels) plus the
per-token entropy and prediction TRL's metrics need. Every row of the batch goes through
`vocab_pass` (head GEMM in the matmul dtype, row kernel, hidden gradient, per group of rows)
with labels -100 ignored. The gradient is taken in the forward (the head is frozen) as
dz @ W with dz = (softmax - onehot) * GRAD_GAIN / denominator stored in the 16-bit matmul
dtype, so that (p - onehot) / num_tokens keeps its precision in fp16; the backward divides
GRAD_GAIN out in fp32 and scales by the incoming loss gradient (solution/cross_entropy.py:
40-44,93-138).

The matmul runs in the autocast dtype, else in promote(hidden, weight) as the reference
chooses it (solution/cross_entropy.py:169). The kernels take fp16 and bf16 only: a direct
call with an fp32 matmul dtype raises TypeError, and the model hook leaves such a model on
its original forward (full logits), as it does every call it does not take.

Hooks (solution/cross_entropy.py:175-321) are built from `head_hooks`: the model forward
answers with the fused loss once armed by the trainer hook, and the trainer hook logs TRL's
entropy / num_tokens / mean_token_accuracy from the per-token statistics.
"""

from __future__ import annotations

import torch

from . import _common, _lib, head_hooks, vocab_pass
from . import gemm as _gemm

IGNORE_INDEX = -100
# rows of logits per chunk (solution/cross_entropy.py:37): as the default argument, the unit of
# the engine's logits budget; passed explicitly, the bound on the live logits
CHUNK_ROWS = vocab_pass.EngineRows(512)
BLOCK_V = 4096  # the reference's vocab block (solution/cross_entropy.py:39); tiles are internal
GRAD_GAIN = 65536.0  # power of two: scaling dz by it and dividing it out in fp32 is exact
STEP_ATTR = head_hooks.STEP_ATTR
VARIANT = "cross_entropy"
MATMUL_DTYPES = (torch.float16, torch.bfloat16)

entropy_from_logits = head_hooks.entropy_from_logits


def _grad_scale(denominator, device):
    """GRAD_GAIN / denominator, or 0 for a zero denominator, as the fp32 scale of dz
    (solution/cross_entropy.py:105-106 forms it on the host from float(denominator)). A
    denominator held on the GPU (the labelled-token count) stays there: the quotient is taken
    in fp64 on the device and rounded to fp32 once, the value the host would pass, without
    the host waiting for the forward to finish."""
    if torch.is_tensor(denominator) and denominator.device == device and device.type == "cuda":
        d = denominator.detach().reshape(()).to(torch.float64)
        return torch.where(d != 0, GRAD_GAIN / d, torch.zeros_like(d)).to(torch.float32).reshape(1)
    divisor = float(denominator)
    return GRAD_GAIN / divisor if divisor else 0.0


class FusedLinearCrossEntropy(torch.autograd.Function):
    """loss = sum over rows of CE(hidden @ W.T, target) / denominator, with per-token loss,
    entropy and argmax, never holding more than one group of rows' logits
    (solution/cross_entropy.py:93-138). W is frozen: only `hidden` gets a gradient."""

    @staticmethod
    def forward(ctx, hidden, weight, target, denominator, matmul_dtype, chunk_rows):
        if matmul_dtype not in MATMUL_DTYPES:
            raise TypeError(f"the fused head loss computes its matmuls in fp16 or bf16, not "
                            f"{matmul_dtype}: enable autocast or give 16-bit hidden states "
                            f"and head weight")
        _lib.require_device(hidden, weight)
        lead, width = hidden.shape[:-1], hidden.shape[-1]
        flat = hidden.reshape(-1, width)
        n = flat.shape[0]
        labels = target.reshape(-1).to(device=hidden.device, dtype=torch.int64).contiguous()
        rows = vocab_pass.RowResults(n, hidden.device, pred=True)
        grad_scale = _grad_scale(denominator, hidden.device)
        grad = None
        if ctx.needs_input_grad[0]:
            grad = torch.empty((n, width), dtype=torch.float32, device=hidden.device)
        with torch.autocast(device_type=hidden.device.type, enabled=False):
            vocab_pass.run(flat.to(matmul_dtype).contiguous(),
                           _gemm.frozen_as(weight, matmul_dtype), labels, rows,
                           ignore_mode=vocab_pass.IGNORE_MINUS_100, chunk_rows=chunk_rows,
                           grad=grad, grad_rows=n if grad is not None else 0,
                           grad_scale=grad_scale)
        ctx.save_for_backward(grad)
        ctx.lead, ctx.dtype = lead, hidden.dtype
        ctx.mark_non_differentiable(rows.loss, rows.entropy, rows.pred)
        return (rows.loss.sum() / denominator, rows.loss.view(lead), rows.entropy.view(lead),
                rows.pred.view(lead))

    @staticmethod
    def backward(ctx, grad_loss, _grad_token_loss, _grad_entropy, _grad_pred):
        (grad,) = ctx.saved_tensors
        if grad is None:
            return None, None, None, None, None, None
        d_hidden = (grad * (grad_loss.float() / GRAD_GAIN)).view(*ctx.lead, -1).to(ctx.dtype)
        return d_hidden, None, None, None, None, None


class ChunkedStep:
    """The per-token results a fused step leaves for the metrics and a rewind recorder:
    token_entropy and token_loss ([B, T], loss 0 where unlabelled), and the labelled and
    correct token counts (solution/cross_entropy.py:141-150)."""

    def __init__(self, token_entropy, token_loss, pred, target):
        self.token_entropy = token_entropy
        self.token_loss = token_loss
        scored = target != IGNORE_INDEX
        self.labelled = scored.sum()
        self.correct = (scored & (pred == target)).sum()


def shift_labels_of(labels):
    """Labels moved one position left with -100 appended, as ForCausalLMLoss shifts them
    (solution/cross_entropy.py:153-155)."""
    tail = torch.full_like(labels[..., :1], IGNORE_INDEX)
    return torch.cat([labels[..., 1:], tail], dim=-1)


def _matmul_dtype(hidden_dtype, weight_dtype):
    return _common.autocast_dtype() or torch.promote_types(hidden_dtype, weight_dtype)


def fused_causal_lm_loss(hidden, weight, labels, num_items_in_batch=None, shift_labels=None,
                         chunk_rows=CHUNK_ROWS):
    """ForCausalLMLoss(hidden @ weight.T, labels) and a ChunkedStep, without the full logits
    (solution/cross_entropy.py:158-172). The divisor is num_items_in_batch when given, else
    the number of labelled tokens (a mean)."""
    target = (shift_labels if shift_labels is not None else shift_labels_of(labels))
    target = target.to(hidden.device)
    if num_items_in_batch is None:
        denominator = (target != IGNORE_INDEX).sum()
    elif torch.is_tensor(num_items_in_batch):
        denominator = num_items_in_batch.to(hidden.device)
    else:
        denominator = num_items_in_batch
    loss, token_loss, entropy, pred = FusedLinearCrossEntropy.apply(
        hidden, weight, target, denominator, _matmul_dtype(hidden.dtype, weight.dtype),
        chunk_rows)
    return loss, ChunkedStep(entropy, token_loss, pred, target)


# ---- hooks (solution/cross_entropy.py:175-321) -----------------------------------------------
class _Armed:
    """`armed` is set by the trainer hook (or a harness) for one model forward; the forward
    disarms it and leaves its ChunkedStep in `step`."""

    armed = False
    step = None


STATE = _Armed()


def _hidden_dtype(lm):
    """The dtype of the decoder's last hidden state: the final norm's output,
    promote(norm weight, residual stream); None when the model does not say."""
    try:
        return torch.promote_types(lm.model.norm.weight.dtype,
                                   lm.model.embed_tokens.weight.dtype)
    except AttributeError:
        return None


def _head_ok(lm):
    """The head of `lm` takes the fused path: a frozen, bias-free Linear on the GPU with no
    logit soft-capping (solution/cross_entropy.py:183-187) whose matmul would run in fp16 or
    bf16 (the kernels' dtypes; anything else keeps the original forward)."""
    if head_hooks.head_refusal(lm) is not None:
        return False
    hidden_dtype = _hidden_dtype(lm)
    return hidden_dtype is None or \
        _matmul_dtype(hidden_dtype, lm.lm_head.weight.dtype) in MATMUL_DTYPES


def _wants(model, labels, logits_to_keep, kwargs):
    return (STATE.armed and labels is not None and _common.on_gpu(labels)
            and head_hooks.plain_training_call(logits_to_keep, kwargs) and _head_ok(model))


def _head_loss(model, hidden, labels, attention_mask, kwargs):
    STATE.armed = False
    loss, STATE.step = fused_causal_lm_loss(hidden, model.lm_head.weight, labels,
                                            num_items_in_batch=kwargs.get("num_items_in_batch"),
                                            shift_labels=kwargs.get("shift_labels"))
    return loss


def _patch_causal_lm():
    """Qwen2ForCausalLM.forward computes the fused loss once armed, else runs the forward it
    wrapped (solution/cross_entropy.py:190-222)."""
    head_hooks.install_model_hook(VARIANT, _wants, _head_loss)


def _causal_lm_of(trainer, model):
    """The Qwen2ForCausalLM under accelerate and peft wrappers
    (solution/cross_entropy.py:225-229)."""
    unwrap = getattr(getattr(trainer, "accelerator", None), "unwrap_model", None)
    return head_hooks.base_model(unwrap(model) if callable(unwrap) else model)


def _lm_fits(lm):
    return head_hooks.is_qwen2_causal_lm(lm) and _head_ok(lm)


_REFUSALS = head_hooks.TRAINER_REFUSALS + (
    ("trainer's model is not training",
     lambda t, m, i: not getattr(getattr(t, "model", None), "training", False)),
    ("labels or mask off the GPU",
     lambda t, m, i: not _common.on_gpu(i["labels"], i["attention_mask"])),
    ("the trainer chunks the head loss itself",
     lambda t, m, i: getattr(t, "_soup_chunked_head_loss", None) is not None),
    ("not a Qwen2 causal LM with a fusable head",
     lambda t, m, i: not _lm_fits(_causal_lm_of(t, m))),
)


def _can_fuse(trainer, model, inputs):
    """Whether this compute_loss call may take the fused head: none of the refusals applies
    (solution/cross_entropy.py:232-256)."""
    return head_hooks.refusal(_REFUSALS, trainer, model, inputs) is None


def _log_metrics(trainer, mode, inputs, step):
    """entropy, num_tokens and mean_token_accuracy as trl 0.29.1 SFTTrainer.compute_loss logs
    them (attention_mask present, no virtual tokens), from the step's per-token statistics;
    num_tokens grows in training only (solution/cross_entropy.py:259-276)."""
    mask = inputs["attention_mask"]
    with torch.no_grad():
        entropy = (step.token_entropy * mask).sum() / mask.sum()
    head_hooks.log_trl_metrics(trainer, mode, mask, entropy, step.correct, step.labelled,
                               count_tokens=mode == "train")


def _armed_loss_for(trainer_cls):
    def armed_loss(trainer, model, inputs, num_items_in_batch):
        mode = "train" if trainer.model.training else "eval"
        labels = inputs["labels"]
        STATE.armed, STATE.step = True, None
        try:
            loss, outputs = super(trainer_cls, trainer).compute_loss(
                model, inputs, return_outputs=True, num_items_in_batch=num_items_in_batch)
        finally:
            STATE.armed = False
        step, STATE.step = STATE.step, None
        if step is None:  # the model kept its own forward: the same metrics from its logits
            with torch.no_grad():
                logits = outputs.logits
                step = ChunkedStep(entropy_from_logits(logits), None, logits.argmax(dim=-1),
                                   shift_labels_of(labels))
            setattr(trainer, STEP_ATTR, None)
        else:
            setattr(trainer, STEP_ATTR, step)
        _log_metrics(trainer, mode, inputs, step)
        return loss, outputs
    return armed_loss


def _patch_trainer(trainer_cls=None):
    """Arm the fused head inside `trainer_cls.compute_loss` (default: trl's SFTTrainer; returns
    False when trl is not importable) and log TRL's metrics from the fused statistics
    (solution/cross_entropy.py:279-316). The loss itself comes from the parent class's
    compute_loss, which calls the model with the labels."""
    trainer_cls = trainer_cls or head_hooks.default_trainer_class()
    if trainer_cls is None:
        return False
    head_hooks.install_trainer_hook(VARIANT, trainer_cls, _can_fuse, _armed_loss_for(trainer_cls))
    return True


def patch(trainer_cls=None):
    """Install the model hook and the trainer hook that arms it (solution/cross_entropy.py:
    319-321); the trainer hook goes on `trainer_cls`, by default trl's SFTTrainer when trl is
    importable (it is not in this image, so only the model hook is installed then)."""
    _patch_causal_lm()
    _patch_trainer(trainer_cls)
