"""CPU oracle of the floating-point kernels (torch, fp32 or fp64 on the CPU).

Test infrastructure only. Each function restates the reference's math and cites it; each is
pinned by tests/test_oracle_ops.py against an installed library routine (transformers'
Qwen2RMSNorm / apply_rotary_pos_emb / ForCausalLMLoss, torch autograd, F.silu,
F.cross_entropy, torch.argmax) or against golden vectors.
"""

from __future__ import annotations

import numpy as np
import torch

from . import philox


# ---- RMSNorm (solution/rmsnorm.py:24-55; solution/test_rmsnorm.py:9-15) ----------------------
def rmsnorm_fwd(x: torch.Tensor, w: torch.Tensor, eps: float):
    """(y, rstd): y = w * (x32 * rsqrt(mean(x32^2) + eps)).to(x.dtype), as Qwen2RMSNorm."""
    h = x.float()
    var = h.pow(2).mean(-1, keepdim=True)
    rstd = torch.rsqrt(var + eps)
    y = w * (h * rstd).to(x.dtype)
    return y, rstd.squeeze(-1)


def rmsnorm_bwd(dy: torch.Tensor, x: torch.Tensor, w: torch.Tensor, rstd: torch.Tensor):
    """dx = r * (g - x * r^2 * mean(g*x)), g = dy*w (solution/rmsnorm.py:52-54), in fp64."""
    g = dy.double() * w.double()
    xd = x.double()
    r = rstd.double().unsqueeze(-1)
    dot = (g * xd).mean(-1, keepdim=True)
    return (r * (g - xd * r * r * dot)).to(x.dtype)


# ---- RoPE (solution/rope.py:3-15,24-62; solution/test_rope.py:9-25) --------------------------
def rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
         backward: bool = False):
    """Rotation of (B, H, S, D) q and k by (B|1, S, D) cos/sin, in fp32, result dtype
    promote(x, cos). forward: o1 = x1c1 - x2s1, o2 = x2c2 + x1s2;
    backward: d1 = g1c1 + g2s2, d2 = g2c2 - g1s1."""
    c = cos.float().unsqueeze(1)
    s = sin.float().unsqueeze(1)
    half = q.shape[-1] // 2
    c1, c2, s1, s2 = c[..., :half], c[..., half:], s[..., :half], s[..., half:]

    def rot(x):
        x32 = x.float()
        x1, x2 = x32[..., :half], x32[..., half:]
        if backward:
            o1, o2 = x1 * c1 + x2 * s2, x2 * c2 - x1 * s1
        else:
            o1, o2 = x1 * c1 - x2 * s1, x2 * c2 + x1 * s2
        return torch.cat([o1, o2], -1).to(torch.promote_types(x.dtype, cos.dtype))

    return rot(q), rot(k)


def qwen_cos_sin(batch: int, seq: int, dim: int, theta: float = 1e6, dtype=torch.float32):
    """Qwen2's rotary tables: cat(freqs, freqs) with inv_freq = theta^(-2i/dim)
    (solution/test_rope.py:17-22)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float) / dim))
    pos = torch.arange(seq, dtype=torch.float)
    emb = torch.cat([torch.outer(pos, inv_freq)] * 2, dim=-1)
    return (emb.cos()[None].expand(batch, -1, -1).to(dtype),
            emb.sin()[None].expand(batch, -1, -1).to(dtype))


# ---- SwiGLU (solution/swiglu.py:15-37) -------------------------------------------------------
def swiglu_fwd(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    g, u = gate.double(), up.double()
    return (g * torch.sigmoid(g) * u).to(gate.dtype)


def swiglu_bwd(grad, gate, up):
    gr, g, u = grad.double(), gate.double(), up.double()
    sg = torch.sigmoid(g)
    dup = gr * g * sg
    dgate = gr * u * sg * (1 + g * (1 - sg))
    return dgate.to(gate.dtype), dup.to(up.dtype)


# ---- LoRA cast / add (solution/lora.py:29-60) -------------------------------------------------
def dropout_scale(x: torch.Tensor, p: float, seed: int, scale: float, out_dtype) -> torch.Tensor:
    x2 = x.reshape(-1, x.shape[-1]).float()
    if p > 0:
        keep = torch.from_numpy(philox.keep_mask(seed, x2.shape[0], x2.shape[1], p))
        v = torch.where(keep, x2 * np.float32(scale), torch.zeros_like(x2))
    else:
        v = x2 * np.float32(scale)
    return v.to(out_dtype).view(x.shape)


def scaled_add(base, lo, scaling):
    """out = base + lo * s computed in fp32 with one rounding (the fused multiply-add of
    solution/lora.py:57-59, where s reaches the kernel as an fp32 argument), then cast to
    promote(base, lo) (solution/lora.py:99-100). Evaluated in fp64: the product of an fp32 (or
    16-bit) lo and an fp32 s is exact there, and rounding the fp64 sum to fp32 equals the single
    rounding of the exact sum unless that sum needs more than 53 bits and its fp64 rounding
    lands on an fp32 halfway point (never the case in the tests, which use operands within 29
    binades of each other)."""
    s = float(np.float32(scaling))
    out_dtype = torch.promote_types(base.dtype, lo.dtype)
    return (base.double() + lo.double() * s).float().to(out_dtype)


# ---- CE rows (solution/fused_ce.py:42-96, solution/cross_entropy.py:48-90) -------------------
def ce_rows(logits: torch.Tensor, target: torch.Tensor, ignore_mode: int = 0,
            grad_scale: float = 1.0):
    """Per row in fp64 from the (16-bit) logits: (loss, entropy, argmax, correct, dz)."""
    z = logits.double()
    t = target.long()
    labelled = (t >= 0) if ignore_mode == 0 else (t != -100)
    lse = torch.logsumexp(z, -1)
    p = torch.softmax(z, -1)
    entropy = lse - (p * z).sum(-1)
    safe = torch.where(labelled, t, torch.zeros_like(t))
    zt = z.gather(1, safe[:, None]).squeeze(1)
    loss = torch.where(labelled, lse - zt, torch.zeros_like(lse))
    argmax = torch.argmax(z, -1)
    correct = (labelled & (argmax == t)).int()
    onehot = torch.zeros_like(z).scatter_(1, safe[:, None], 1.0) * labelled[:, None].double()
    dz = (p - onehot) * (labelled.double() * grad_scale)[:, None]
    return loss, entropy, argmax, correct, dz


def shift_labels(labels: torch.Tensor) -> torch.Tensor:
    return torch.nn.functional.pad(labels, (0, 1), value=-100)[..., 1:]


def fused_linear_ce(hidden, weight, labels, num_items_in_batch, matmul_dtype):
    """What the unfused run computes (solution/test_cross_entropy.py:9-29, with TRL's entropy
    restated as lse - sum(p*z)): logits in the matmul dtype, loss on their fp32 upcast.
    Returns (loss, token_entropy, token_loss, pred, correct, labelled, logits)."""
    # a 16-bit matmul with fp32 accumulation, its output rounded to the matmul dtype
    logits = (hidden.to(matmul_dtype).float() @ weight.to(matmul_dtype).float().t())
    logits = logits.to(matmul_dtype).float()
    shift = shift_labels(labels)
    flat, tgt = logits.view(-1, logits.shape[-1]), shift.reshape(-1)
    if num_items_in_batch is None:
        loss = torch.nn.functional.cross_entropy(flat, tgt, ignore_index=-100)
    else:
        loss = torch.nn.functional.cross_entropy(flat, tgt, ignore_index=-100,
                                                 reduction="sum") / num_items_in_batch
    with torch.no_grad():
        z = logits.double()
        lse = torch.logsumexp(z, -1)
        entropy = (lse - (torch.softmax(z, -1) * z).sum(-1)).float()
        token_loss = torch.nn.functional.cross_entropy(
            flat, tgt, ignore_index=-100, reduction="none").view(shift.shape)
        pred = logits.argmax(-1)
        mask = shift != -100
        correct = ((pred == shift) & mask).sum()
    return loss, entropy, token_loss, pred, correct, mask.sum(), logits
