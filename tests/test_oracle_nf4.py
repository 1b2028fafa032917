"""Pins of the NF4 dequant oracle (oracle/nf4_oracle.c, oracle/nf4.py) — CPU only.

Each check is chosen so a plausible mistake fails it: a swapped nibble order, a wrong block
index, a fused multiply-add in the scale, a wrong codebook entry, a wrong bf16 rounding.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from hackathon_amd import quant
from oracle import nf4 as onf4

GOLDEN = Path(__file__).resolve().parent / "golden"
TABLE = np.array(quant.NF4_CODE, dtype=np.float32)


def test_codebook_is_the_published_table():
    published = json.loads((GOLDEN / "nf4_codebook.json").read_text())["values"]
    assert list(quant.NF4_CODE) == published
    # each entry is exactly representable in fp32 (the table is an fp32 table)
    assert [float(np.float32(v)) for v in published] == published


def test_codebook_rederived_from_normal_quantiles():
    """QLoRA construction: 8 positive and 7 negative N(0,1) quantiles + 0, scaled to [-1, 1]."""
    from scipy.stats import norm

    offset = 0.9677083
    pos = norm.ppf(np.linspace(offset, 0.5, 9)[:-1])
    neg = -norm.ppf(np.linspace(offset, 0.5, 8)[:-1])
    v = np.sort(np.concatenate([pos, [0.0], neg]))
    v = v / v.max()
    assert np.abs(v - TABLE.astype(np.float64)).max() < 2e-7


def _kat_state():
    # two blocks of 4 weights; nested scales chosen exactly representable
    code2 = np.zeros(256, np.float32)
    code2[3], code2[200] = 0.5, -0.25
    return dict(absmax=np.array([3, 200], np.uint8), nested=1, code2=code2,
                absmax2=np.array([0.25], np.float32), offset=np.float32(0.0625), blocksize=4,
                blocksize2=256)


def test_known_answer_bytes():
    """Byte 0xF0: weight 0 = nf4[15]*s, weight 1 = nf4[0]*s (high nibble first,
    solution/nf4.py:30,45-47); block 0 scale = 0.5*0.25 + 0.0625 = 0.1875;
    block 1 scale = -0.25*0.25 + 0.0625 = 0.0 (scale order: multiply, then add)."""
    st = _kat_state()
    packed = np.array([0xF0, 0x7F, 0x0F, 0xF8], np.uint8)
    out = onf4.dequant(packed, 8, TABLE, out="f32", **st)
    s0 = np.float32(0.1875)
    expect = np.array([1.0 * s0, -1.0 * s0, 0.0, 1.0 * s0, 0.0, 0.0, 0.0, 0.0], np.float32)
    np.testing.assert_array_equal(out, expect)
    # a block scale off by one block would have used s1 = 0 for weights 2..3: check a block-1
    # weight with a non-zero scale instead
    st["code2"][200] = 1.0  # block 1 scale = 0.25 + 0.0625 = 0.3125
    out = onf4.dequant(packed, 8, TABLE, out="f32", **st)
    assert out[4] == np.float32(-1.0) * np.float32(0.3125)
    assert out[5] == np.float32(TABLE[15] * np.float32(0.3125))
    assert out[6] == np.float32(TABLE[15] * np.float32(0.3125))
    assert out[7] == np.float32(TABLE[8] * np.float32(0.3125))


def test_scale_is_two_roundings_not_an_fma():
    """code2*absmax2 + offset with separate fp32 roundings (what bitsandbytes computes);
    these operands give a different fp32 result under a single-rounding FMA."""
    c, a, off = np.float32(1.0 + 2**-12), np.float32(1.0 + 2**-12), np.float32(-1.0)
    two_round = np.float32(np.float32(c * a) + off)
    fused = np.float32(np.float64(c) * np.float64(a) + np.float64(off))
    assert two_round != fused
    code2 = np.zeros(256, np.float32)
    code2[1] = c
    st = dict(absmax=np.array([1], np.uint8), nested=1, code2=code2,
              absmax2=np.array([a], np.float32), offset=off, blocksize=2, blocksize2=256)
    got = onf4.scales(1, **st)[0]
    assert got == two_round


def test_invariants_on_random_states():
    rng = np.random.default_rng(0)
    n, bs = 64 * 40, 64
    st = dict(absmax=rng.integers(0, 256, n // bs).astype(np.uint8), nested=1,
              code2=np.sort(rng.standard_normal(256)).astype(np.float32),
              absmax2=rng.random(1).astype(np.float32) + 0.5, offset=np.float32(0.03),
              blocksize=bs, blocksize2=256)
    packed = rng.integers(0, 256, n // 2).astype(np.uint8)
    out = onf4.dequant(packed, n, TABLE, out="f32", **st)
    s = onf4.scales(n // bs, **st)
    j = np.arange(n)
    nib = np.where(j & 1, packed[j >> 1] & 15, packed[j >> 1] >> 4)
    blk_s = s[j // bs]
    assert np.all(out[nib == 7] == 0.0)
    np.testing.assert_array_equal(out[nib == 15], blk_s[nib == 15])
    np.testing.assert_array_equal(out[nib == 0], -blk_s[nib == 0])
    # monotone in the nibble for a positive scale, antitone for a negative one
    for b in range(n // bs):
        seg = out[b * bs:(b + 1) * bs]
        ns = nib[b * bs:(b + 1) * bs]
        order = np.argsort(ns, kind="stable")
        d = np.diff(seg[order])
        assert np.all(d >= 0) if s[b] >= 0 else np.all(d <= 0)
    # the numpy twin agrees bit-for-bit on the fp32 result
    np.testing.assert_array_equal(onf4.dequant_numpy(packed, n, TABLE, **st), out)


def test_plain_absmax_reduces_to_codebook_times_absmax():
    rng = np.random.default_rng(1)
    n, bs = 128 * 10, 128
    absmax = rng.random(n // bs).astype(np.float32)
    packed = rng.integers(0, 256, n // 2).astype(np.uint8)
    out = onf4.dequant(packed, n, TABLE, absmax=absmax, nested=0, code2=None, absmax2=None,
                       offset=0.0, blocksize=bs, blocksize2=1, out="f32")
    codes = torch.from_numpy(np.stack([packed >> 4, packed & 15], 1).reshape(-1).astype(np.int64))
    expect = (torch.from_numpy(TABLE)[codes].view(-1, bs) * torch.from_numpy(absmax)[:, None])
    np.testing.assert_array_equal(out, expect.reshape(-1).numpy())


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(2)
    specials = np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 1.0 + 2**-8, 1.0 + 3 * 2**-8,
                         3.4e38, -3.4e38, 1e-40, -1e-40, 2**-126, np.inf, -np.inf], np.float32)
    ties = (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    vals = np.concatenate([specials, ties, rng.standard_normal(5000).astype(np.float32) * 0.02])
    ours = onf4.f32_to_bf16_bits(vals)
    theirs = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


@pytest.mark.parametrize("nested", [True, False])
def test_quantise_dequantise_quantise_is_idempotent(nested):
    """Re-quantising dequantised weights reproduces the codes; a wrong nibble order or block
    index in dequant (or in the packing) breaks this."""
    g = torch.Generator().manual_seed(0)
    w = torch.randn(96, 320, generator=g) * 0.02
    packed, st = quant.quantize_nf4(w, 64, compress_statistics=nested)
    deq = onf4.dequant_state(packed, st, TABLE, out="f32").reshape(96, 320)
    packed2, _ = quant.quantize_nf4(torch.from_numpy(deq), 64, compress_statistics=False)
    assert torch.equal(packed, packed2)


def test_dequant_error_is_bounded_by_half_the_code_gap():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(64, 256, generator=g) * 0.02
    packed, st = quant.quantize_nf4(w, 64, compress_statistics=False)
    deq = onf4.dequant_state(packed, st, TABLE, out="f32").reshape(64, 256)
    half_gap = np.max(np.diff(TABLE)) / 2
    absmax = w.reshape(-1, 64).abs().amax(1).repeat_interleave(64).reshape(64, 256).numpy()
    assert np.all(np.abs(deq - w.numpy()) <= absmax * half_gap * (1 + 1e-5))


@pytest.mark.parametrize("shape,nested", [((4864, 896), True), ((7, 50), True), ((96, 320), False)])
def test_torch_restatement_matches_the_c_oracle(shape, nested):
    """The vectorised torch dequant (the CPU baseline) equals the C oracle bit for bit, on the
    Qwen2.5-0.5B gate_proj weight and on a ragged shape whose last block is partial."""
    g = torch.Generator().manual_seed(3)
    w = torch.randn(shape, generator=g) * 0.02
    packed, st = quant.quantize_nf4(w, 64, compress_statistics=nested)
    want = onf4.dequant_state(packed, st, TABLE, out="bf16")
    got = onf4.dequant_torch(packed, st, TABLE)
    np.testing.assert_array_equal(got.view(torch.int16).numpy().view(np.uint16), want)
