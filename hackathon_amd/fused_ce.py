"""The output head and the loss without the full logits tensor, with row selection: drop-in
for solution/fused_ce.py (the variant that keeps only the rows a training step needs).

`fused_head_loss` computes transformers' ForCausalLMLoss(lm_head(hidden), labels) and the
per-row statistics TRL's metrics need, through `vocab_pass` (head GEMM, row kernel, hidden
gradient per group of rows, the head in fp16 as the reference's autocast run has it):

  - the rows of the pass are the positions with a label, then the real positions without one
    (entropy only), each in position order; padding positions are left out. The order comes
    from one stable sort of a per-position rank (0 labelled, 1 real unlabelled, 2 padding);
  - the hidden gradient is taken in the forward for the labelled rows only, divided by the
    loss's denominator; backward only scales it (the head is frozen);
  - per-position loss and entropy are scattered back to [batch, seq] for the trainer hook
    (TRL's metrics) and for a rewind recorder (`token_loss`).

The model and trainer hooks (solution/fused_ce.py:222-355) are built from `head_hooks`.
"""

from __future__ import annotations

import torch

from . import _lib, head_hooks, vocab_pass
from . import gemm as _gemm

# rows of logits per chunk (solution/fused_ce.py:33): left as it is, the unit of the engine's
# logits budget; set to another value (a plain int, 512 included), the bound on the live logits
CHUNK = vocab_pass.EngineRows(512)
IGNORE = -100
STEP_ATTR = head_hooks.STEP_ATTR
VARIANT = "fused_ce"

_LABELLED, _UNLABELLED, _PADDING = 0, 1, 2


def ce_rows(logits, target, write_grad):
    """Per-row loss, entropy and correct flag of [n, vocab] logits; with write_grad the logits
    are overwritten by softmax - onehot (solution/fused_ce.py:99-109). Rows with a negative
    target are unlabelled."""
    _lib.require_device(logits, target)
    if logits.stride(-1) != 1:
        raise ValueError("logits rows must be unit-stride")
    out = vocab_pass.RowResults(logits.shape[0], logits.device, correct=True)
    vocab_pass.row_statistics(logits, target.to(torch.int64).contiguous(), out, 0,
                              vocab_pass.IGNORE_NEGATIVE, write_grad, 1.0)
    return out.loss, out.entropy, out.correct


class FusedLinearCE(torch.autograd.Function):
    """Rows of hidden states [n, hidden] -> sum of their cross-entropies / denominator, and the
    per-row loss, entropy and correct flag (solution/fused_ce.py:112-158). Rows [0, n_labelled)
    carry a label; the others only feed the metrics. weight16 is the frozen fp16 head."""

    @staticmethod
    def forward(ctx, hidden, weight16, target, n_labelled, denominator):
        _lib.require_device(hidden, weight16)
        n, width = hidden.shape
        rows = vocab_pass.RowResults(n, hidden.device, correct=True)
        grad = None
        if ctx.needs_input_grad[0]:
            grad = torch.zeros((n, width), dtype=torch.float32, device=hidden.device)
        with torch.autocast(hidden.device.type, enabled=False):
            vocab_pass.run(hidden.to(weight16.dtype).contiguous(), weight16.contiguous(),
                           target.to(torch.int64).contiguous(), rows,
                           ignore_mode=vocab_pass.IGNORE_NEGATIVE, chunk_rows=CHUNK, grad=grad,
                           grad_rows=int(n_labelled))
        if grad is not None:
            ctx.save_for_backward(grad.div_(denominator))
        ctx.mark_non_differentiable(rows.loss, rows.entropy, rows.correct)
        return rows.loss.sum() / denominator, rows.loss, rows.entropy, rows.correct

    @staticmethod
    def backward(ctx, grad_total, _loss, _entropy, _correct):
        (grad,) = ctx.saved_tensors
        return grad * grad_total, None, None, None, None


class Stats:
    """What `fused_head_loss` reports beside the loss: token_loss [batch, seq] (0 off the
    labelled positions), entropy_sum over the real positions, and the correct and labelled
    token counts (0-dim tensors)."""

    __slots__ = ("token_loss", "entropy_sum", "correct", "labelled")

    def __init__(self, token_loss, entropy_sum, correct, labelled):
        self.token_loss, self.entropy_sum = token_loss, entropy_sum
        self.correct, self.labelled = correct, labelled


class _Step:
    """What a rewind recorder reads for a step without logits: the per-token loss."""

    __slots__ = ("token_loss",)

    def __init__(self, token_loss):
        self.token_loss = token_loss


def _row_order(targets, attention_mask):
    """(rows, n_labelled): the positions the pass runs, labelled ones first, then real
    unlabelled ones, each group in position order (one stable sort of the rank)."""
    rank = torch.full_like(targets, _UNLABELLED)
    if attention_mask is not None:
        rank.masked_fill_(attention_mask.reshape(-1) == 0, _PADDING)
    rank.masked_fill_(targets != IGNORE, _LABELLED)
    order = torch.sort(rank, stable=True).indices
    n_labelled, n_unlabelled, _ = torch.bincount(rank, minlength=3).tolist()
    return order[: n_labelled + n_unlabelled], n_labelled


def _denominator(num_items_in_batch, n_labelled, device):
    """ForCausalLMLoss's divisor: num_items_in_batch when given (a tensor moves to the
    device), else the number of labelled positions (a mean)."""
    if num_items_in_batch is None:
        return torch.tensor(float(n_labelled), device=device)
    if torch.is_tensor(num_items_in_batch):
        return num_items_in_batch.to(device)
    return num_items_in_batch


def fused_head_loss(hidden, weight, labels, attention_mask, num_items_in_batch):
    """ForCausalLMLoss(hidden @ weight.T, labels) and a Stats for TRL's metrics, without the
    logits (solution/fused_ce.py:178-219). hidden [batch, seq, width]; labels [batch, seq]
    are shifted here (position t is scored against labels[t + 1])."""
    batch, seq, width = hidden.shape
    device = hidden.device
    targets = torch.cat([labels.to(device)[:, 1:],
                         torch.full((batch, 1), IGNORE, dtype=labels.dtype, device=device)],
                        dim=1).reshape(-1)
    if attention_mask is not None:
        attention_mask = attention_mask.to(device)
    rows, n_labelled = _row_order(targets, attention_mask)
    denominator = _denominator(num_items_in_batch, n_labelled, device)
    # the fp16 head (solution/fused_ce.py:202), cast once per frozen weight and kept while the
    # weight is unchanged, so its transpose for dz @ W is kept with it
    head = _gemm.frozen_as(weight, torch.float16)
    loss, row_loss, row_entropy, row_correct = FusedLinearCE.apply(
        hidden.reshape(-1, width)[rows], head, targets[rows], n_labelled, denominator)
    with torch.no_grad():
        per_position = torch.zeros((2, batch * seq), dtype=torch.float32, device=device)
        per_position[:, rows] = torch.stack((row_loss, row_entropy))
        token_loss, token_entropy = per_position
        if attention_mask is not None:
            token_entropy = token_entropy * attention_mask.reshape(-1)
        stats = Stats(token_loss=token_loss.view(batch, seq), entropy_sum=token_entropy.sum(),
                      correct=row_correct[:n_labelled].sum(),
                      labelled=torch.tensor(n_labelled, device=device))
    return loss, stats


# ---- hooks (solution/fused_ce.py:222-355) ----------------------------------------------------
class _Armed:
    """Set by the trainer hook around exactly one model forward; the forward leaves its Stats."""

    active = False
    stats = None


STATE = _Armed()
_HEAD_DTYPES = (torch.float32, torch.float16)


def _head_fits(causal_lm):
    """A Qwen2 causal LM whose lm_head is a frozen, bias-free fp32 or fp16 Linear on the GPU
    with no logit soft-capping (solution/fused_ce.py:236-246)."""
    return (head_hooks.is_qwen2_causal_lm(causal_lm)
            and head_hooks.head_refusal(causal_lm, _HEAD_DTYPES) is None)


_REFUSALS = head_hooks.TRAINER_REFUSALS + (
    ("model is not training", lambda t, m, i: not m.training),
    ("head does not fit", lambda t, m, i: not _head_fits(head_hooks.base_model(m))),
)


def _can_fuse(trainer, model, inputs):
    """Whether a compute_loss call takes the fused head: none of the trainer refusals applies
    and the (peft-unwrapped) model is a Qwen2 causal LM whose head fits
    (solution/fused_ce.py:285-303)."""
    return head_hooks.refusal(_REFUSALS, trainer, model, inputs) is None


def _wants(model, labels, logits_to_keep, kwargs):
    return (STATE.active and labels is not None and model.training
            and head_hooks.plain_training_call(logits_to_keep, kwargs)
            and kwargs.get("shift_labels") is None and _head_fits(model))


def _head_loss(model, hidden, labels, attention_mask, kwargs):
    loss, STATE.stats = fused_head_loss(hidden, model.lm_head.weight, labels, attention_mask,
                                        kwargs.get("num_items_in_batch"))
    return loss


def patch_qwen2_causal_lm():
    """Qwen2ForCausalLM.forward answers with `fused_head_loss` (no logits) when the trainer hook
    is active and the call is a plain training forward with labels; any other call runs the
    forward it wrapped (solution/fused_ce.py:249-282)."""
    head_hooks.install_model_hook(VARIANT, _wants, _head_loss)


def _armed_loss(trainer, model, inputs, num_items_in_batch):
    from transformers import Trainer

    STATE.active, STATE.stats = True, None
    try:
        loss, outputs = Trainer.compute_loss(trainer, model, inputs, return_outputs=True,
                                             num_items_in_batch=num_items_in_batch)
    finally:
        STATE.active = False
    stats, STATE.stats = STATE.stats, None
    if stats is None:
        raise RuntimeError("hackathon_amd: the fused head loss did not run in this step")
    mask = inputs["attention_mask"]
    head_hooks.log_trl_metrics(trainer, "train", mask, stats.entropy_sum / mask.sum(),
                               stats.correct, stats.labelled, count_tokens=True)
    setattr(trainer, STEP_ATTR, _Step(stats.token_loss))
    return loss, outputs


def _forget_step(trainer):
    if getattr(trainer, STEP_ATTR, None) is not None:
        setattr(trainer, STEP_ATTR, None)


_HOOKED = []  # trainer classes whose compute_loss this variant wraps


def patch_sft_trainer(trainer_cls=None):
    """Activate the fused head inside `trainer_cls.compute_loss` (default: trl's SFTTrainer;
    returns False when trl is not importable), log TRL's metrics from the fused statistics and
    leave the per-token loss under STEP_ATTR (solution/fused_ce.py:306-355)."""
    trainer_cls = trainer_cls or head_hooks.default_trainer_class()
    if trainer_cls is None:
        return False
    head_hooks.install_trainer_hook(VARIANT, trainer_cls, _can_fuse, _armed_loss,
                                    on_fallback=_forget_step)
    if trainer_cls not in _HOOKED:
        _HOOKED.append(trainer_cls)
    return True


def unpatch():
    """Remove this variant's model and trainer hooks."""
    head_hooks.remove_model_hook(VARIANT)
    while _HOOKED:
        head_hooks.remove_trainer_hook(VARIANT, _HOOKED.pop())
