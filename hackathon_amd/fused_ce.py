"""The output head and the loss without the full logits tensor (drop-in for solution/fused_ce.py).

Per training forward (solution/fused_ce.py:8-19):
1. only the positions that matter are kept, labelled rows first, then real unlabelled rows
   (for the entropy metric); padding is dropped;
2. the head runs on CHUNK rows at a time into one reused [CHUNK, vocab] buffer
   (qlora_gemm, fp16 operands as the reference's autocast run);
3. one workgroup per row reads the row of logits and computes logsumexp, the cross-entropy at
   the label, the entropy and the argmax; a second sweep overwrites the logits in place with
   softmax - onehot (qlora_ce_rows);
4. the hidden-state gradient dz @ W is taken right there, chunk by chunk (qlora_gemm into an
   fp32 buffer), so nothing of vocabulary size outlives its chunk; backward only scales it.
"""

from __future__ import annotations

import torch

from . import _lib
from . import gemm as _gemm

CHUNK = 512  # rows of logits alive at a time (solution/fused_ce.py:33)
IGNORE = -100
STEP_ATTR = "_soup_chunked_step"


def ce_rows(logits, target, write_grad):
    """Per-row loss, entropy and correct flag of [n, vocab] logits; with write_grad the logits
    are overwritten by softmax - onehot (solution/fused_ce.py:99-109)."""
    _lib.require_device(logits, target)
    n, vocab = logits.shape
    if logits.stride(-1) != 1:
        raise ValueError("logits rows must be unit-stride")
    target = target.to(torch.int64).contiguous()
    loss = torch.empty(n, dtype=torch.float32, device=logits.device)
    entropy = torch.empty(n, dtype=torch.float32, device=logits.device)
    correct = torch.empty(n, dtype=torch.int32, device=logits.device)
    if n:
        _lib.call("qlora_ce_rows", logits.data_ptr(), _lib.tag(logits.dtype), logits.stride(0),
                  n, vocab, target.data_ptr(), loss.data_ptr(), entropy.data_ptr(),
                  correct.data_ptr(), None, 0, int(bool(write_grad)), 1.0,
                  _lib.stream_of(logits))
    return loss, entropy, correct


def _head_gemm(h, w, out):
    """logits chunk = h @ w.T into `out` (MFMA kernel for 16-bit operands)."""
    if h.dtype in (torch.float16, torch.bfloat16):
        _gemm.gemm(h, w, out=out)
    else:
        torch.mm(h, w.t(), out=out)


def _grad_gemm(dz, w, out):
    """out (fp32) = dz @ w, run as dz @ (w^T)^T against the cached transpose of the frozen
    head weight, so both operands are k-contiguous (the vocabulary is the reduction)."""
    if dz.dtype in (torch.float16, torch.bfloat16):
        _gemm.gemm(dz, _gemm.transposed_frozen(w), out=out)
    else:
        out.copy_(torch.mm(dz, w))


class FusedLinearCE(torch.autograd.Function):
    """Rows of hidden states [n, hidden] -> sum of their cross-entropies / denominator
    (solution/fused_ce.py:112-158). Rows [0, n_labelled) have a label; the head is frozen and
    the hidden gradient is computed in forward and only scaled in backward."""

    @staticmethod
    def forward(ctx, hidden, weight16, target, n_labelled, denominator):
        n, width = hidden.shape
        vocab = weight16.shape[0]
        with_grad = ctx.needs_input_grad[0]
        hidden16 = hidden.to(weight16.dtype).contiguous()
        weight16 = weight16.contiguous()
        grad = torch.zeros((n, width), dtype=torch.float32, device=hidden.device) \
            if with_grad else None
        buffer = _gemm.padded_rows(min(CHUNK, max(n, 1)), vocab, weight16.dtype, hidden.device)
        losses, entropies, corrects = [], [], []
        with torch.autocast(hidden.device.type, enabled=False):
            for start in range(0, n, CHUNK):
                stop = min(n, start + CHUNK)
                logits = buffer[: stop - start]
                _head_gemm(hidden16[start:stop], weight16, logits)
                labelled = max(0, min(stop, n_labelled) - start)
                write_grad = with_grad and labelled > 0
                loss, entropy, correct = ce_rows(logits, target[start:stop], write_grad)
                losses.append(loss)
                entropies.append(entropy)
                corrects.append(correct)
                if write_grad:
                    _grad_gemm(logits[:labelled], weight16, grad[start:start + labelled])
        del buffer
        row_loss = torch.cat(losses) if losses else hidden.new_zeros(0, dtype=torch.float32)
        row_entropy = torch.cat(entropies) if entropies else row_loss
        row_correct = torch.cat(corrects) if corrects else row_loss.int()
        total = row_loss.sum() / denominator
        if with_grad:
            grad /= denominator
            ctx.save_for_backward(grad)
        ctx.mark_non_differentiable(row_loss, row_entropy, row_correct)
        return total, row_loss, row_entropy, row_correct

    @staticmethod
    def backward(ctx, grad_total, _l, _e, _c):
        (grad,) = ctx.saved_tensors
        return grad * grad_total, None, None, None, None


class Stats:
    __slots__ = ("token_loss", "entropy_sum", "correct", "labelled")

    def __init__(self, token_loss, entropy_sum, correct, labelled):
        self.token_loss, self.entropy_sum = token_loss, entropy_sum
        self.correct, self.labelled = correct, labelled


class _Step:
    """What a trainer's per-row loss recorder reads for a step without logits."""

    __slots__ = ("token_loss",)

    def __init__(self, token_loss):
        self.token_loss = token_loss


def fused_head_loss(hidden, weight, labels, attention_mask, num_items_in_batch):
    """ForCausalLMLoss(lm_head(hidden), labels) and TRL's metrics without the logits
    (solution/fused_ce.py:178-219)."""
    batch, seq, width = hidden.shape
    device = hidden.device
    labels = labels.to(device)
    target = torch.nn.functional.pad(labels, (0, 1), value=IGNORE)[:, 1:].reshape(-1)
    has_label = target != IGNORE
    if attention_mask is None:
        real = torch.ones_like(has_label)
    else:
        real = attention_mask.to(device).reshape(-1) != 0
    other = real & ~has_label
    label_rows = has_label.nonzero().squeeze(1)
    other_rows = other.nonzero().squeeze(1)
    rows = torch.cat([label_rows, other_rows])
    n_labelled = label_rows.numel()

    if num_items_in_batch is None:
        denominator = torch.tensor(float(n_labelled), device=device)
    elif torch.is_tensor(num_items_in_batch):
        denominator = num_items_in_batch.to(device)
    else:
        denominator = num_items_in_batch

    weight16 = weight if weight.dtype == torch.float16 else weight.detach().to(torch.float16)
    picked = hidden.reshape(-1, width).index_select(0, rows)
    loss, row_loss, row_entropy, row_correct = FusedLinearCE.apply(
        picked, weight16, target.index_select(0, rows), n_labelled, denominator)

    with torch.no_grad():
        token_loss = torch.zeros(batch * seq, dtype=torch.float32, device=device)
        token_loss.index_copy_(0, rows, row_loss)
        token_entropy = torch.zeros(batch * seq, dtype=torch.float32, device=device)
        token_entropy.index_copy_(0, rows, row_entropy)
        if attention_mask is None:
            entropy_sum = token_entropy.sum()
        else:
            entropy_sum = (token_entropy * attention_mask.to(device).reshape(-1)).sum()
        stats = Stats(token_loss=token_loss.view(batch, seq), entropy_sum=entropy_sum,
                      correct=row_correct[:n_labelled].sum(),
                      labelled=torch.tensor(n_labelled, device=device))
    return loss, stats
