"""Pins of the floating-point oracle (oracle/ops.py) and the dropout oracle (oracle/philox.py)
against installed library routines and golden vectors — CPU only."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import ops, philox

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---- RMSNorm ------------------------------------------------------------------------------------
@pytest.mark.parametrize("x_dtype,w_dtype", [(torch.float32, torch.float32),
                                              (torch.bfloat16, torch.bfloat16),
                                              (torch.float16, torch.float32)])
def test_rmsnorm_forward_is_qwen2rmsnorm(x_dtype, w_dtype):
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    g = torch.Generator().manual_seed(0)
    norm = Qwen2RMSNorm(1536, eps=1e-6)
    norm.weight.data = (1 + 0.1 * torch.randn(1536, generator=g)).to(w_dtype)
    x = torch.randn(3, 7, 1536, generator=g).to(x_dtype)
    y, rstd = ops.rmsnorm_fwd(x, norm.weight.data, 1e-6)
    want = norm(x)
    assert y.dtype == want.dtype
    torch.testing.assert_close(y, want, rtol=0, atol=0)
    torch.testing.assert_close(rstd, torch.rsqrt(x.float().pow(2).mean(-1) + 1e-6))


def test_rmsnorm_backward_closed_form_is_autograd():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 1000, generator=g, dtype=torch.float64)
    w = 1 + 0.1 * torch.randn(1000, generator=g, dtype=torch.float64)
    dy = torch.randn(5, 1000, generator=g, dtype=torch.float64)
    xr = x.clone().requires_grad_()
    rstd = torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + 1e-6)
    (w * xr * rstd * dy).sum().backward()
    got = ops.rmsnorm_bwd(dy, x, w, rstd.detach().squeeze(-1))
    torch.testing.assert_close(got, xr.grad, rtol=1e-12, atol=1e-12)


# ---- RoPE ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("batch_cos", [1, 3])
def test_rope_forward_is_apply_rotary_pos_emb(batch_cos):
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    g = torch.Generator().manual_seed(0)
    B, S, HQ, HK, D = 3, 11, 12, 2, 128
    q = torch.randn(B, S, HQ, D, generator=g).transpose(1, 2)
    k = torch.randn(B, S, HK, D, generator=g).transpose(1, 2)
    cos, sin = ops.qwen_cos_sin(batch_cos, S, D)
    qo, ko = ops.rope(q, k, cos, sin)
    rq, rk = apply_rotary_pos_emb(q, k, cos, sin)
    torch.testing.assert_close(qo, rq, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(ko, rk, rtol=1e-6, atol=1e-6)


def test_rope_backward_is_the_autograd_transpose_with_unequal_halves():
    """General cos/sin (halves differ): the backward formula is the vector-Jacobian product of
    q*cos + rotate_half(q)*sin, which autograd computes independently."""
    g = torch.Generator().manual_seed(2)
    B, S, H, D = 2, 5, 3, 16
    q = torch.randn(B, H, S, D, generator=g, dtype=torch.float64, requires_grad=True)
    cos = torch.randn(B, S, D, generator=g, dtype=torch.float64)
    sin = torch.randn(B, S, D, generator=g, dtype=torch.float64)
    gq = torch.randn(B, H, S, D, generator=g, dtype=torch.float64)

    def rotate_half(x):
        return torch.cat((-x[..., D // 2:], x[..., :D // 2]), -1)

    (q * cos.unsqueeze(1) + rotate_half(q) * sin.unsqueeze(1)).mul(gq).sum().backward()
    got, _ = ops.rope(gq.float(), gq.float(), cos.float(), sin.float(), backward=True)
    torch.testing.assert_close(got.double(), q.grad, rtol=1e-5, atol=1e-5)


# ---- SwiGLU -------------------------------------------------------------------------------------
def test_swiglu_is_silu_times_up_with_autograd_backward():
    g = torch.Generator().manual_seed(0)
    gate = torch.randn(4, 77, generator=g, dtype=torch.float64, requires_grad=True)
    up = torch.randn(4, 77, generator=g, dtype=torch.float64, requires_grad=True)
    grad = torch.randn(4, 77, generator=g, dtype=torch.float64)
    ref = torch.nn.functional.silu(gate) * up
    ref.backward(grad)
    torch.testing.assert_close(ops.swiglu_fwd(gate.detach(), up.detach()), ref.detach())
    dg, du = ops.swiglu_bwd(grad, gate.detach(), up.detach())
    torch.testing.assert_close(dg, gate.grad)
    torch.testing.assert_close(du, up.grad)


# ---- dropout uniform (Philox) -------------------------------------------------------------------
def test_philox_known_answer_vectors():
    kat = json.loads((GOLDEN / "philox_kat.json").read_text())
    for case in kat["cases"]:
        ctr = [np.uint32(int(v, 16)) for v in case["ctr"]]
        key = [np.uint32(int(v, 16)) for v in case["key"]]
        out = philox.philox4x32_10(*ctr, *key)
        assert [f"{int(o):08x}" for o in out] == case["out"]


def test_uniform_matches_tritons_tl_rand():
    data = json.loads((GOLDEN / "triton_rand.json").read_text())
    for case in data["cases"]:
        got = philox.uniform(case["seed"], np.array(case["offsets"], dtype=np.int64))
        assert got.view(np.int32).tolist() == case["bits"], case["seed"]


def test_dropout_oracle_rate_scale_and_determinism():
    x = torch.randn(64, 1536)
    y = ops.dropout_scale(x, 0.05, 1234, 1 / 0.95, torch.float32)
    kept = y != 0
    assert abs((1 - kept.float().mean().item()) - 0.05) < 0.01
    torch.testing.assert_close(y[kept], (x * np.float32(1 / 0.95))[kept], rtol=0, atol=0)
    assert torch.equal(ops.dropout_scale(x, 0.05, 1234, 1 / 0.95, torch.float32) != 0, kept)
    assert not torch.equal(ops.dropout_scale(x, 0.05, 4321, 1 / 0.95, torch.float32) != 0, kept)
    # p = 0 is a plain cast
    torch.testing.assert_close(ops.dropout_scale(x, 0.0, 0, 1.0, torch.bfloat16),
                               x.to(torch.bfloat16), rtol=0, atol=0)


# ---- cross-entropy ------------------------------------------------------------------------------
@pytest.mark.parametrize("ignore_mode", [0, 1])
def test_ce_rows_against_cross_entropy_and_brute_force(ignore_mode):
    g = torch.Generator().manual_seed(0)
    z = (torch.randn(9, 1001, generator=g) * 3).to(torch.bfloat16)
    t = torch.randint(0, 1001, (9,), generator=g)
    t[2] = -100
    z[4, 17] = z[4].max() + 1   # a clear argmax
    z[5, 3] = z[5, 800] = z[5].max() + 1  # a tie: the first index wins
    loss, ent, am, correct, dz = ops.ce_rows(z, t, ignore_mode, grad_scale=2.0)
    zf = z.double()
    want = torch.nn.functional.cross_entropy(zf, t, ignore_index=-100, reduction="none")
    torch.testing.assert_close(loss, want)
    p = torch.softmax(zf, -1)
    torch.testing.assert_close(ent, -(p * torch.log(p)).sum(-1))
    assert am[4] == 17 and am[5] == 3
    assert torch.equal(am, torch.argmax(zf, -1))
    assert correct.tolist() == [int(t[i] >= 0 and am[i] == t[i]) for i in range(9)]
    # dz is the gradient of sum(loss)*grad_scale w.r.t. z
    zr = zf.clone().requires_grad_()
    (torch.nn.functional.cross_entropy(zr, t, ignore_index=-100, reduction="sum") * 2.0).backward()
    torch.testing.assert_close(dz, zr.grad)


def test_fused_linear_ce_oracle_is_forcausallmloss():
    from transformers.loss.loss_utils import ForCausalLMLoss

    g = torch.Generator().manual_seed(0)
    b, t, h, v = 2, 9, 32, 500
    hidden = torch.randn(b, t, h, generator=g)
    weight = 0.05 * torch.randn(v, h, generator=g)
    labels = torch.randint(0, v, (b, t), generator=g)
    labels[:, :3] = -100
    items = (labels[:, 1:] != -100).sum()
    loss, ent, tok, pred, correct, lab, logits = ops.fused_linear_ce(
        hidden, weight, labels, items, torch.float32)
    want = ForCausalLMLoss(logits, labels, v, num_items_in_batch=items)
    torch.testing.assert_close(loss, want)
    assert int(lab) == int(items)
    # the per-token losses sum to the total
    torch.testing.assert_close(tok.sum() / items, want)


# ---- scaled add: pinned against exact rational arithmetic ------------------------------------
def _round_f32(x):
    """The fp32 value nearest the rational x, ties to even (IEEE 754 round-to-nearest), from
    the definition: 24 significand bits for normal numbers, a quantum of 2^-149 below."""
    from fractions import Fraction

    if x == 0:
        return 0.0
    sign, x = (-1.0 if x < 0 else 1.0), abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    q = max(e - 23, -149)
    scaled = x / Fraction(2) ** q
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * n * 2.0 ** q


def _exact_scaled_add(base, lo, scaling, out_dtype):
    """base + lo * fp32(scaling) evaluated exactly, rounded once to fp32, then cast."""
    from fractions import Fraction

    s = Fraction(float(np.float32(scaling)))
    vals = [_round_f32(Fraction(float(b)) + Fraction(float(v)) * s)
            for b, v in zip(base.reshape(-1).tolist(), lo.reshape(-1).tolist())]
    return torch.tensor(vals, dtype=torch.float32).view(base.shape).to(out_dtype)


@pytest.mark.parametrize("base_dtype,lo_dtype", [(torch.float32, torch.float16),
                                                 (torch.float32, torch.bfloat16),
                                                 (torch.bfloat16, torch.bfloat16),
                                                 (torch.float16, torch.float32),
                                                 (torch.float32, torch.float32)])
@pytest.mark.parametrize("scaling", [2.0, 0.5, 3.0, 0.3])
def test_scaled_add_is_one_fp32_rounding_then_the_promoted_cast(base_dtype, lo_dtype, scaling):
    g = torch.Generator().manual_seed(7)
    base = torch.randn(3, 67, generator=g).to(base_dtype)
    lo = (torch.randn(3, 67, generator=g) * 4).to(lo_dtype)
    out_dtype = torch.promote_types(base_dtype, lo_dtype)
    got = ops.scaled_add(base, lo, scaling)
    assert got.dtype == out_dtype
    assert torch.equal(got, _exact_scaled_add(base, lo, scaling, out_dtype))


def test_scaled_add_crafted_cases():
    f32 = torch.float32
    # one rounding, not two: (1 + 2^-12)^2 - (1 + 2^-11) = 2^-24 exactly; rounding the product
    # to fp32 first (a tie, to even) would give 0
    a = torch.tensor([1 + 2.0 ** -12], dtype=f32)
    got = ops.scaled_add(torch.tensor([-(1 + 2.0 ** -11)], dtype=f32), a, 1 + 2.0 ** -12)
    assert got.item() == 2.0 ** -24
    # fp32 arithmetic for 16-bit lo: 65504 * 2 overflows fp16 but not fp32
    got = ops.scaled_add(torch.tensor([0.5], dtype=f32), torch.tensor([65504.0]).half(), 2.0)
    assert got.dtype == f32 and got.item() == 131008.5
    # the scaling multiplies lo only: s = 0 returns base, and base is never scaled
    base = torch.tensor([1.5, -2.25, 3.0], dtype=f32)
    lo = torch.tensor([7.0, 9.0, -1.0]).half()
    assert torch.equal(ops.scaled_add(base, lo, 0.0), base)
    assert ops.scaled_add(base, lo, 2.0).tolist() == [15.5, 15.75, 1.0]
    # s reaches the kernel as fp32: 0.3 is 0.30000001192..., visible in an fp32 result
    got = ops.scaled_add(torch.tensor([0.0], dtype=f32), torch.tensor([2.0 ** 20], dtype=f32), 0.3)
    assert got.item() == float(np.float32(0.3)) * 2.0 ** 20
    # a 16-bit output is rounded from the fp32 result, not from the exact sum: 1 + 2^-8 + 2^-30
    # rounds to fp32 1 + 2^-8, a bf16 halfway point that ties to even (1.0), while rounding the
    # exact sum straight to bf16 would give 1 + 2^-7
    bf = torch.bfloat16
    got = ops.scaled_add(torch.tensor([1.0], dtype=bf), torch.tensor([2.0 ** -8], dtype=bf),
                         1 + 2.0 ** -22)
    assert got.dtype == bf and got.item() == 1.0
    # the exact reference agrees on every case above
    for b, v, s, dt in (([-(1 + 2.0 ** -11)], [1 + 2.0 ** -12], 1 + 2.0 ** -12, f32),
                        ([0.5], [3.0], 2.0, f32), ([1.0], [2.0 ** -8], 1 + 2.0 ** -22, bf)):
        bt, vt = torch.tensor(b, dtype=dt), torch.tensor(v, dtype=dt)
        assert torch.equal(ops.scaled_add(bt, vt, s), _exact_scaled_add(bt, vt, s, dt))


@pytest.mark.parametrize("batch,seq,dim,theta,dtype", [(1, 2048, 128, 1e6, torch.float32),
                                                        (2, 77, 64, 1e4, torch.bfloat16),
                                                        (1, 512, 128, 1e6, torch.float16)])
def test_qwen_cos_sin_is_qwen2_rotary_embedding(batch, seq, dim, theta, dtype):
    """The oracle's rotary tables equal transformers' Qwen2RotaryEmbedding (the tables the
    model feeds RoPE) for the same head dim, theta and positions 0 .. seq - 1, in every dtype."""
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding

    cfg = Qwen2Config(hidden_size=dim * 4, num_attention_heads=4, num_key_value_heads=2,
                      rope_theta=theta, max_position_embeddings=max(seq, 32))
    rot = Qwen2RotaryEmbedding(cfg)
    x = torch.zeros(batch, seq, dim, dtype=dtype)
    pos = torch.arange(seq)[None].expand(batch, -1)
    want_cos, want_sin = rot(x, pos)
    cos, sin = ops.qwen_cos_sin(batch, seq, dim, theta=theta, dtype=dtype)
    assert cos.shape == want_cos.shape and cos.dtype == want_cos.dtype
    assert torch.equal(cos, want_cos) and torch.equal(sin, want_sin)
