"""Rows of hidden states through a frozen output head and the cross-entropy, without the logits
of the whole batch: the engine both fused lm_head + CE variants run on (`fused_ce.FusedLinearCE`,
`cross_entropy.FusedLinearCrossEntropy`; the reference's chunk loops are
solution/fused_ce.py:131-143 and solution/cross_entropy.py:113-124).

For each group of rows, three launches on the stream of the hidden states:

  1. z = h @ W^T               qlora_gemm_ws, the MFMA NT GEMM, z in the 16-bit matmul dtype
  2. row statistics of z       qlora_ce_rows: loss, entropy, argmax (or correct flag); then,
                               when a gradient is wanted, z is overwritten IN PLACE by
                               dz = (softmax(z) - onehot(label)) * scale
  3. grad_h = dz @ W           qlora_gemm_ws against the cached W^T (the vocabulary is the
                               contiguous reduction), fp32 out, for the rows that need it

Grouping. The reference bounds the live logits at `chunk_rows` rows (512 x 151936 x 2 B =
155 MB). An MI355X has 288 GB of HBM, so with the callers' default chunk size (`EngineRows`,
the value 512 marked as the default) the engine runs as many whole chunks per GEMM as fit
`LOGITS_BUDGET` bytes of logits (still a fixed bound, independent of the batch): W (467 MB at
151936 x 1536 bf16) is streamed once per group rather than once per chunk, and dz @ W becomes
one tall GEMM instead of sixteen skinny split-K ones. A chunk size a caller passes explicitly
(any plain int, 512 included) is the reference's hard bound: groups of at most that many rows.
The groups are balanced and the row count of each a multiple of 256 (one GEMM tile) where
possible. Per-row results do not depend on the grouping: each row's statistics come from its
own logits, and each row of grad_h from its own dz.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from . import gemm as _gemm

# 1.25 GiB of live logits per group: 4096 rows at the Qwen2 vocabulary, so a batch of 8192
# tokens never holds all its logits at once. Measured on MI355X at 8192 x 1536 x 151936
# (forward + dz @ W): one group of 8192 rows 7.84-8.33 ms, two of 4096 7.95-7.99 ms, four of
# 2048 8.13-8.27 ms, eight of 1024 8.97-9.11 ms.
LOGITS_BUDGET = 5 << 28
TILE_ROWS = 256          # the NT GEMM's M tile



class EngineRows(int):
    """The reference's default chunk size (512 rows) as the façades' default argument: passed
    as is, the engine groups whole chunks up to LOGITS_BUDGET; any other value, a plain 512
    included, bounds the live logits at that many rows, as solution/cross_entropy.py:37-38 and
    solution/fused_ce.py:33 do."""

    def __repr__(self):
        return int.__repr__(self)


def budget_for(chunk_rows):
    """Bytes of live logits a group may hold for this chunk argument: LOGITS_BUDGET for the
    default (EngineRows), else 0, which plan_groups turns into one chunk per group."""
    return LOGITS_BUDGET if isinstance(chunk_rows, EngineRows) else 0


IGNORE_NEGATIVE = 0      # a row is labelled when its target is >= 0 (solution/fused_ce.py:48)
IGNORE_MINUS_100 = 1     # a row is labelled when its target is not -100 (cross_entropy.py:54)


class RowResults:
    """Per-row outputs of one pass, allocated once for every row: fp32 `loss` (0 for an
    unlabelled row) and `entropy`, and either the int32 `correct` flag (labelled and argmax ==
    label) or the int64 `pred` (argmax, first index of the maximum)."""

    __slots__ = ("loss", "entropy", "correct", "pred")

    def __init__(self, n, device, *, correct=False, pred=False):
        self.loss = torch.empty(n, dtype=torch.float32, device=device)
        self.entropy = torch.empty(n, dtype=torch.float32, device=device)
        self.correct = torch.empty(n, dtype=torch.int32, device=device) if correct else None
        self.pred = torch.empty(n, dtype=torch.int64, device=device) if pred else None

    def pointers(self, start):
        """Device addresses of row `start` in each output (None for an absent output)."""
        def at(t):
            return None if t is None else t.data_ptr() + start * t.element_size()
        return at(self.loss), at(self.entropy), at(self.correct), at(self.pred)


def plan_groups(n_rows, vocab, chunk_rows, elem_bytes=2, budget=LOGITS_BUDGET):
    """[(start, stop)] row ranges covering n_rows: whole multiples of `chunk_rows` up to
    `budget` bytes of logits per group (at least one chunk), balanced across the groups and
    rounded up to whole GEMM tiles."""
    if n_rows <= 0:
        return []
    chunk_rows = max(1, int(chunk_rows))
    per_chunk = chunk_rows * vocab * elem_bytes
    cap = chunk_rows * max(1, budget // max(per_chunk, 1))
    n_groups = math.ceil(n_rows / cap)
    size = math.ceil(n_rows / n_groups)
    tiled = math.ceil(size / TILE_ROWS) * TILE_ROWS
    if tiled <= cap:
        size = tiled
    return [(a, min(a + size, n_rows)) for a in range(0, n_rows, size)]


def row_statistics(logits, target, out, start, ignore_mode, write_grad, grad_scale):
    """qlora_ce_rows over one group's logits [rows, vocab] (16-bit or fp32, unit stride along
    the vocabulary), filling rows start.. of `out`; with write_grad the logits become
    dz = (softmax - onehot) * (labelled ? grad_scale : 0) in place. `grad_scale` is a number,
    or a one-element fp32 tensor on the device that the kernel reads there
    (qlora_ce_rows_scale_ptr), so a scale formed on the GPU costs the host no wait."""
    rows, vocab = logits.shape
    if rows == 0:
        return
    loss, entropy, correct, pred = out.pointers(start)
    if torch.is_tensor(grad_scale):
        if (grad_scale.dtype != torch.float32 or grad_scale.numel() != 1
                or grad_scale.device != logits.device):
            raise ValueError("a tensor grad_scale must be one fp32 value on the logits' device")
        _lib.call("qlora_ce_rows_scale_ptr", logits.data_ptr(), _lib.tag(logits.dtype),
                  logits.stride(0), rows, vocab, target.data_ptr(), loss, entropy, correct, pred,
                  ignore_mode, int(bool(write_grad)), grad_scale.data_ptr(),
                  _lib.stream_of(logits))
        return
    _lib.call("qlora_ce_rows", logits.data_ptr(), _lib.tag(logits.dtype), logits.stride(0), rows,
              vocab, target.data_ptr(), loss, entropy, correct, pred, ignore_mode,
              int(bool(write_grad)), float(grad_scale), _lib.stream_of(logits))


def run(hidden, weight, target, out, *, ignore_mode, chunk_rows, grad=None, grad_rows=0,
        grad_scale=1.0):
    """One pass of `hidden` [n, H] (the matmul dtype, unit stride along H) through the frozen
    head `weight` [V, H] (same dtype): per-row statistics into `out` (a RowResults of n rows)
    and, when `grad` (fp32 [n, H]) is given, grad[r] = dz[r] @ W for the rows r < grad_rows;
    rows from grad_rows on are left untouched in `grad`. `target` is int64 [n] on the device.
    `grad_scale` is a number or a one-element fp32 device tensor (row_statistics).
    `chunk_rows`: an EngineRows lets groups grow to LOGITS_BUDGET; a plain int is the bound on
    the rows of live logits."""
    n, vocab = hidden.shape[0], weight.shape[0]
    if hidden.dtype != weight.dtype or weight.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("the head GEMMs take fp16 or bf16 operands of one dtype, got "
                        f"{hidden.dtype} and {weight.dtype}")
    groups = plan_groups(n, vocab, chunk_rows, weight.element_size(), budget_for(chunk_rows))
    if not groups:
        return
    want_grad = grad is not None and grad_rows > 0
    buffer = _gemm.padded_rows(max(b - a for a, b in groups), vocab, weight.dtype, hidden.device)
    weight_t = _gemm.transposed_frozen(weight) if want_grad else None
    for a, b in groups:
        logits = buffer[: b - a]
        _gemm.gemm(hidden[a:b], weight, out=logits)
        grad_stop = min(b, grad_rows) if want_grad else a
        row_statistics(logits, target[a:b], out, a, ignore_mode, grad_stop > a, grad_scale)
        if grad_stop > a:
            _gemm.gemm(logits[: grad_stop - a], weight_t, out=grad[a:grad_stop])
