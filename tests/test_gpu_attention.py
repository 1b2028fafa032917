"""Flash attention on the GPU vs an fp32 reference of causal softmax attention with grouped
query heads (torch fp32 products on the GPU, transposed operands made contiguous first).
Tolerances: output within rtol = atol = 1e-2 (bf16), log-sum-exp within 1e-4."""

import math

import pytest
import torch

from hackathon_amd import attention

pytestmark = pytest.mark.gpu


def _ref(q, k, v, scale):
    """fp32 causal attention: (o [B, HQ, S, D], lse [B, HQ, S])."""
    B, HQ, S, D = q.shape
    rep = HQ // k.shape[1]
    kf = k.float().repeat_interleave(rep, dim=1)
    vf = v.float().repeat_interleave(rep, dim=1)
    s = torch.matmul(q.float(), kf.transpose(-1, -2).contiguous()) * scale
    mask = torch.ones(S, S, dtype=torch.bool, device=q.device).triu(1)
    s = s.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vf), lse


def _inputs(B, HQ, HK, S, seed, layout="bshd"):
    g = torch.Generator(device="cuda").manual_seed(seed)
    D = 128
    if layout == "bshd":  # (B, H, S, D) views of (B, S, H, D) buffers, as Qwen2Attention makes
        q = torch.randn(B, S, HQ, D, device="cuda", generator=g).to(torch.bfloat16).transpose(1, 2)
        k = torch.randn(B, S, HK, D, device="cuda", generator=g).to(torch.bfloat16).transpose(1, 2)
        v = torch.randn(B, S, HK, D, device="cuda", generator=g).to(torch.bfloat16).transpose(1, 2)
    else:
        q = torch.randn(B, HQ, S, D, device="cuda", generator=g).to(torch.bfloat16)
        k = torch.randn(B, HK, S, D, device="cuda", generator=g).to(torch.bfloat16)
        v = torch.randn(B, HK, S, D, device="cuda", generator=g).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("B,HQ,HK,S,layout", [(1, 4, 2, 256, "bshd"), (1, 2, 1, 200, "bhsd"),
                                              (2, 28, 4, 2048, "bshd"), (1, 3, 3, 64, "bhsd")])
def test_flash_attention_forward(B, HQ, HK, S, layout):
    print(f"attn fwd B={B} HQ={HQ} HK={HK} S={S} {layout}", flush=True)
    q, k, v = _inputs(B, HQ, HK, S, seed=S + HQ, layout=layout)
    scale = 1.0 / math.sqrt(128)
    o, lse = attention.attn_fwd(q, k, v, scale)
    o_ref, lse_ref = _ref(q, k, v, scale)
    assert o.shape == (B, S, HQ, 128)
    torch.testing.assert_close(o.transpose(1, 2).float(), o_ref, rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(lse, lse_ref, rtol=0, atol=1e-4)
