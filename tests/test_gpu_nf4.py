"""NF4 dequant on the GPU vs the C oracle: bit-exact for bf16 and fp32 outputs."""

import numpy as np
import pytest
import torch

from hackathon_amd import nf4, quant
from oracle import nf4 as onf4
from tests._util import bits16

pytestmark = pytest.mark.gpu
TABLE = np.array(quant.NF4_CODE, dtype=np.float32)


def _case(shape, nested, blocksize, seed=0):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(shape, generator=g) * 0.02
    packed, st = quant.quantize_nf4(w, blocksize, compress_statistics=nested)
    want_bf16 = onf4.dequant_state(packed, st, TABLE, out="bf16")
    want_f32 = onf4.dequant_state(packed, st, TABLE, out="f32")
    return packed.cuda(), st.to("cuda"), want_bf16, want_f32


@pytest.mark.parametrize("shape,nested,blocksize", [
    ((4864, 896), True, 64),      # Qwen2.5-0.5B gate_proj, double quant
    ((4864, 896), False, 64),
    ((96, 320), True, 64),
    ((256, 1536), True, 128),
    ((33, 64), True, 32),
    ((7, 6), True, 64),           # fewer bytes than one vector group: scalar tail only
    ((3, 10), False, 64),
    ((13, 18), True, 6),          # even, non power-of-two blocksize: scalar kernel
])
def test_dequant_bit_exact(shape, nested, blocksize):
    print(f"nf4 dequant {shape} nested={nested} bs={blocksize}", flush=True)
    packed, st, want_bf16, want_f32 = _case(shape, nested, blocksize)
    out = nf4.dequantize_nf4(packed, st, torch.bfloat16)
    assert out.shape == shape and out.dtype == torch.bfloat16
    np.testing.assert_array_equal(bits16(out).cpu().numpy().reshape(-1).view(np.uint16), want_bf16)
    out32 = nf4.dequantize_nf4(packed, st, torch.float32)
    np.testing.assert_array_equal(out32.cpu().numpy().reshape(-1), want_f32)
    out16 = nf4.dequantize_nf4(packed, st, torch.float16)
    assert torch.equal(bits16(out16).cpu(),
                       bits16(torch.from_numpy(want_f32).to(torch.float16)).view(shape))


def test_dequant_unaligned_buffers_take_the_exact_path():
    print("nf4 dequant unaligned", flush=True)
    packed, st, want_bf16, _ = _case((64, 96), True, 64, seed=5)
    big = torch.zeros(packed.numel() + 1, dtype=torch.uint8, device="cuda")
    big[1:] = packed.reshape(-1)
    out_big = torch.empty(64 * 96 + 1, dtype=torch.bfloat16, device="cuda")
    out = out_big[1:].view(64, 96)                      # 2-byte aligned only
    nf4.dequantize_nf4(big[1:], st, torch.bfloat16, out=out)
    np.testing.assert_array_equal(bits16(out).cpu().numpy().reshape(-1).view(np.uint16), want_bf16)


def test_dequant_full_qwen25_7b_gate_shape_bit_exact():
    """18944 x 3584 (the gate/up projection of the 7B step), the full weight."""
    print("nf4 dequant 18944x3584", flush=True)
    packed, st, want_bf16, _ = _case((18944, 3584), True, 64, seed=7)
    out = nf4.dequantize_nf4(packed, st, torch.bfloat16)
    got = bits16(out).cpu().numpy().reshape(-1).view(np.uint16)
    np.testing.assert_array_equal(got, want_bf16)


@pytest.mark.parametrize("shape,dtype,nested,bs", [
    ((128, 512), torch.float32, True, 64),
    ((18944, 3584), torch.bfloat16, True, 64),   # Qwen2.5-7B gate_proj, as the step builds it
    ((96, 320), torch.float16, False, 64),
    ((33, 70), torch.float32, True, 6),           # partial last block, odd blocksize multiple
    ((7, 6), torch.bfloat16, True, 64),           # fewer weights than one block
    ((65, 130), torch.bfloat16, True, 128),       # partial last block of the lane-shared path
    ((40, 24), torch.float16, False, 16),         # two lanes a block
    ((96, 96), torch.float32, True, 512),         # 64 lanes a block, a partial last block
])
def test_quantizer_kernel_matches_cpu_bytes(shape, dtype, nested, bs):
    """The GPU quantiser kernel and the CPU torch quantiser give identical packed codes, absmax
    codes, second-level scales and offset (the offset is an fp64-accumulated mean)."""
    print(f"nf4 quantize {shape} {dtype} nested={nested} bs={bs}", flush=True)
    g = torch.Generator().manual_seed(11)
    w = (torch.randn(shape, generator=g) * 0.02).to(dtype)
    p_cpu, s_cpu = quant.quantize_nf4(w, bs, compress_statistics=nested)
    p_gpu, s_gpu = quant.quantize_nf4(w.cuda(), bs, compress_statistics=nested)
    assert torch.equal(p_cpu, p_gpu.cpu())
    assert torch.equal(s_cpu.absmax, s_gpu.absmax.cpu())
    if nested:
        assert torch.equal(s_cpu.offset, s_gpu.offset.cpu())
        assert torch.equal(s_cpu.state2.absmax, s_gpu.state2.absmax.cpu())
        assert torch.equal(s_cpu.state2.code, s_gpu.state2.code.cpu())


@pytest.mark.parametrize("nested", [False, True])
def test_quantizer_codes_at_bucket_edges_and_midpoints(nested):
    """The GPU quantiser finds each code through a 256-bucket table (floor(128 v) picks the
    bucket, one midpoint at most per bucket). Products exactly on a bucket edge or an NF4
    midpoint, and one ulp either side, give the CPU quantiser's bytes: every block holds 1.0
    (absmax 1, so v is the weight itself) and 63 such values."""
    print(f"nf4 quantize edges nested={nested}", flush=True)
    code = np.array(quant.NF4_CODE, dtype=np.float32)
    mids = ((code[:-1] + code[1:]) * np.float32(0.5)).astype(np.float32)
    edges = (np.arange(257, dtype=np.float32) / np.float32(128) - np.float32(1)).astype(np.float32)
    pts = np.concatenate([edges, mids, np.float32([0.0, -0.0])])
    vals = np.concatenate([pts, np.nextafter(pts, np.float32(-2)), np.nextafter(pts, np.float32(2))])
    vals = np.clip(vals, -1, 1).astype(np.float32)
    vals = np.concatenate([vals, np.zeros((-len(vals)) % 63, np.float32)]).reshape(-1, 63)
    w = torch.from_numpy(np.concatenate([np.ones((len(vals), 1), np.float32), vals], axis=1))
    p_cpu, s_cpu = quant.quantize_nf4(w, 64, compress_statistics=nested)
    p_gpu, s_gpu = quant.quantize_nf4(w.cuda(), 64, compress_statistics=nested)
    assert torch.equal(p_cpu, p_gpu.cpu())
    assert torch.equal(s_cpu.absmax, s_gpu.absmax.cpu())


@pytest.mark.parametrize("shape,nested,blocksize", [
    ((384, 256), True, 64),
    ((136, 512), True, 64),       # a partial 64-row tile
    ((512, 3584), False, 64),
    ((264, 1024), True, 128),
    ((3584, 18944), True, 64),    # Qwen2.5-7B down_proj
])
def test_transposed_dequant_bit_exact(shape, nested, blocksize):
    """dequantize_nf4_t writes W^T with the same bits as the oracle's W, transposed."""
    print(f"nf4 dequant_t {shape} nested={nested} bs={blocksize}", flush=True)
    packed, st, want_bf16, _ = _case(shape, nested, blocksize, seed=5)
    assert nf4.transposed_dequant_ok(st)
    out_t = nf4.dequantize_nf4_t(packed, st, torch.bfloat16)
    assert out_t.shape == (shape[1], shape[0])
    want_t = want_bf16.reshape(shape).T
    np.testing.assert_array_equal(bits16(out_t).cpu().numpy().view(np.uint16), want_t)


def _concat_rows(outs_shapes, dtype):
    rows = sum(r for r, _ in outs_shapes)
    w = torch.empty((rows, outs_shapes[0][1]), dtype=dtype, device="cuda")
    offs = np.cumsum([0] + [r for r, _ in outs_shapes])
    return w, [w[offs[i]:offs[i + 1]] for i in range(len(outs_shapes))], offs


@pytest.mark.parametrize("shapes,nested,blocksize,dtype", [
    ([(96, 320), (40, 320), (8, 320)], True, 64, torch.bfloat16),
    ([(64, 256), (72, 256), (128, 256), (8, 256)], False, 128, torch.float32),
    ([(3584, 3584), (512, 3584), (512, 3584)], True, 64, torch.bfloat16),  # Qwen2.5-7B q/k/v
])
def test_grouped_dequant_bit_exact(shapes, nested, blocksize, dtype):
    """One qlora_nf4_dequant_group launch writes every weight with the oracle's bits."""
    print(f"nf4 dequant group {shapes} nested={nested} bs={blocksize} {dtype}", flush=True)
    cases = [_case(sh, nested, blocksize, seed=20 + i) for i, sh in enumerate(shapes)]
    w, outs, _ = _concat_rows(shapes, dtype)
    items = [(c[0], c[1]) for c in cases]
    assert nf4._groupable(items, outs, False)
    nf4.dequantize_nf4_group(items, dtype, outs)
    for c, out in zip(cases, outs):
        if dtype == torch.float32:
            np.testing.assert_array_equal(out.cpu().numpy().reshape(-1), c[3])
        else:
            np.testing.assert_array_equal(bits16(out).cpu().numpy().reshape(-1).view(np.uint16),
                                          c[2])


@pytest.mark.parametrize("shapes,nested,blocksize", [
    ([(128, 256), (64, 256), (72, 256)], True, 64),       # a partial 64-row tile
    ([(64, 512), (136, 256)], False, 64),                 # narrower second weight
    ([(3584, 3584), (512, 3584), (512, 3584)], True, 64),  # Qwen2.5-7B q/k/v
])
def test_grouped_transposed_dequant_bit_exact(shapes, nested, blocksize):
    """One qlora_nf4_dequant_t_group launch writes each W_i^T into its column block of a shared
    [in_features, sum out_features] buffer with the oracle's bits, and leaves the rest alone."""
    print(f"nf4 dequant_t group {shapes} nested={nested} bs={blocksize}", flush=True)
    cases = [_case(sh, nested, blocksize, seed=30 + i) for i, sh in enumerate(shapes)]
    kmax = max(c for _, c in shapes)
    offs = np.cumsum([0] + [r for r, _ in shapes])
    sentinel = torch.full((kmax, int(offs[-1])), 7.0, dtype=torch.bfloat16, device="cuda")
    wt = sentinel.clone()
    outs = [wt[:c, offs[i]:offs[i + 1]] for i, (_, c) in enumerate(shapes)]
    items = [(c[0], c[1]) for c in cases]
    assert nf4._groupable(items, outs, True)
    nf4.dequantize_nf4_t_group(items, torch.bfloat16, outs)
    for (r, c), case, out in zip(shapes, cases, outs):
        want_t = case[2].reshape(r, c).T
        np.testing.assert_array_equal(bits16(out).cpu().numpy().view(np.uint16), want_t)
    mask = torch.ones_like(wt, dtype=torch.bool)
    for i, (_, c) in enumerate(shapes):
        mask[:c, offs[i]:offs[i + 1]] = False
    assert torch.equal(wt[mask], sentinel[mask])


def test_grouped_dequant_falls_back_for_mixed_nesting():
    """Weights of different nesting are dequantised one launch each, with the same bits."""
    print("nf4 dequant group mixed nesting", flush=True)
    a = _case((64, 256), True, 64, seed=40)
    b = _case((32, 256), False, 64, seed=41)
    items = [(a[0], a[1]), (b[0], b[1])]
    _, outs, _ = _concat_rows([(64, 256), (32, 256)], torch.bfloat16)
    assert not nf4._groupable(items, outs, False)
    nf4.dequantize_nf4_group(items, torch.bfloat16, outs)
    for c, out in zip((a, b), outs):
        np.testing.assert_array_equal(bits16(out).cpu().numpy().reshape(-1).view(np.uint16), c[2])
