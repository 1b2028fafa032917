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


def patch():
    """Install the model hook (solution/cross_entropy.py:319-321 also patches trl's
    SFTTrainer.compute_loss to arm it; trl is not part of this package's scope)."""
    _patch_causal_lm()
