"""The MFMA GEMM vs an fp64 CPU product of the same 16-bit inputs.

With fp32 accumulation over K terms of magnitude ~|a||b|, the error bound used is
  |C - C_ref| <= 2^-22 * K * max|a| * max|b| * 4  + (one rounding of the output dtype).
"""

import pytest
import torch

from hackathon_amd import gemm

pytestmark = pytest.mark.gpu


def _ref(a, b, a_km, b_kn):
    A = a.double().t() if a_km else a.double()
    B = b.double() if b_kn else b.double().t()
    return A @ B


def _check(out, ref, K, a, b, out_dtype):
    bound = 4 * 2.0**-22 * K * a.abs().max().item() * b.abs().max().item()
    if out_dtype != torch.float32:
        eps = 2.0**-8 if out_dtype == torch.bfloat16 else 2.0**-11
        bound = bound + eps * ref.abs()
    err = (out.double().cpu() - ref).abs()
    assert torch.all(err <= bound + 1e-30), (err - bound).max().item()


@pytest.mark.parametrize("M,N,K", [(256, 384, 512), (130, 250, 72), (1, 3, 8), (4096, 16, 3584),
                                   (16, 4096, 16), (777, 129, 1000), (1024, 640, 768)])
@pytest.mark.parametrize("a_km,b_kn", [(False, False), (False, True), (True, True), (True, False)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_layouts(M, N, K, a_km, b_kn, dtype):
    print(f"gemm M={M} N={N} K={K} a_km={a_km} b_kn={b_kn} {dtype}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    a = torch.randn((K, M) if a_km else (M, K), generator=g).to(dtype)
    b = torch.randn((K, N) if b_kn else (N, K), generator=g).to(dtype)
    for out_dtype in (dtype, torch.float32):
        out = gemm.gemm(a.cuda(), b.cuda(), a_km=a_km, b_kn=b_kn, out_dtype=out_dtype)
        _check(out, _ref(a, b, a_km, b_kn), K, a, b, out_dtype)


def test_gemm_bias_alpha_beta():
    g = torch.Generator().manual_seed(9)
    M, N, K = 200, 300, 256
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    b = torch.randn(N, K, generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    c0 = torch.randn(M, N, generator=g)
    out = c0.clone().cuda()
    gemm.gemm(a.cuda(), b.cuda(), out=out, bias=bias.cuda(), alpha=0.5, beta=2.0)
    ref = 0.5 * (a.double() @ b.double().t()) + 2.0 * c0.double() + bias.double()
    _check(out, ref, K, a, b, torch.float32)


def test_linear_and_matmul_helpers_match_torch_shapes():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 3, 64, generator=g).to(torch.bfloat16).cuda()
    w = torch.randn(48, 64, generator=g).to(torch.bfloat16).cuda()
    y = gemm.linear(x, w)
    assert y.shape == (2, 3, 48) and y.dtype == torch.bfloat16
    torch.testing.assert_close(y.float(), (x.float() @ w.float().t()), rtol=1e-2, atol=1e-2)
    dy = torch.randn(2, 3, 48, generator=g).to(torch.bfloat16).cuda()
    dx = gemm.matmul_nn(dy, w)
    assert dx.shape == (2, 3, 64)
    torch.testing.assert_close(dx.float(), dy.float() @ w.float(), rtol=1e-2, atol=1e-2)


def test_gemm_output_view_with_row_stride():
    """An output chunk that is a row slice of a bigger buffer (as the CE chunk loop writes)."""
    g = torch.Generator().manual_seed(5)
    a = torch.randn(96, 64, generator=g).to(torch.bfloat16)
    b = torch.randn(160, 64, generator=g).to(torch.bfloat16)
    buf = torch.zeros(200, 160, device="cuda")
    gemm.gemm(a.cuda(), b.cuda(), out=buf[50:146])
    _check(buf[50:146], a.double() @ b.double().t(), 64, a, b, torch.float32)
    assert torch.all(buf[:50] == 0) and torch.all(buf[146:] == 0)


@pytest.mark.parametrize("M,N,K", [(512, 768, 1024), (300, 520, 192), (257, 255, 64),
                                   (1000, 3000, 640), (300, 448, 128), (1000, 3584, 640),
                                   (4096, 3584, 256), (4000, 3584, 128), (4096, 4608, 192),
                                   (4000, 4608, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_nt_large_tile_edges(M, N, K, dtype):
    """k-contiguous operands with K % 64 == 0 take the large-tile kernel (256 x 256, or
    256 x 224 when N is a multiple of 224 and it fills the CUs better: the 4096 and 4000 x 3584
    cases take 224, the 4000-row ones with a ragged last row of tiles); M and N edges are
    loaded clamped and must never be stored."""
    print(f"gemm_nt M={M} N={N} K={K} {dtype}", flush=True)
    g = torch.Generator().manual_seed(M + 11 * N + K)
    a = torch.randn(M, K, generator=g).to(dtype)
    b = torch.randn(N, K, generator=g).to(dtype)
    ref = a.double() @ b.double().t()
    for out_dtype in (dtype, torch.float32):
        buf = torch.full((M + 2, N + 8), 7.0, dtype=out_dtype, device="cuda")
        out = buf[1:M + 1, 4:N + 4]
        gemm.gemm(a.cuda(), b.cuda(), out=out)
        _check(out, ref, K, a, b, out_dtype)
        assert torch.all(buf[0] == 7) and torch.all(buf[M + 1] == 7)
        assert torch.all(buf[:, :4] == 7) and torch.all(buf[:, N + 4:] == 7)


@pytest.mark.parametrize("N", [320, 448])
def test_gemm_nt_bias_alpha_beta_large_tile(N):
    g = torch.Generator().manual_seed(19 + N)
    M, K = 384, 256
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    b = torch.randn(N, K, generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    c0 = torch.randn(M, N, generator=g)
    out = c0.clone().cuda()
    gemm.gemm(a.cuda(), b.cuda(), out=out, bias=bias.cuda(), alpha=-1.5, beta=0.25)
    ref = -1.5 * (a.double() @ b.double().t()) + 0.25 * c0.double() + bias.double()
    _check(out, ref, K, a, b, torch.float32)


@pytest.mark.parametrize("M,N,K", [(256, 256, 8192), (512, 1536, 30464), (4096, 512, 3584),
                                   (100, 70, 4096), (256, 3584, 8192)])
def test_gemm_split_k_matches_and_is_deterministic(M, N, K):
    """Small outputs with long K are split over K into an fp32 workspace and summed in split
    order: the result is within the fp32-accumulation bound and identical run to run."""
    from hackathon_amd import _lib

    print(f"gemm split-K M={M} N={N} K={K}", flush=True)
    assert _lib.load().qlora_gemm_workspace_size(0, 0, M, N, K) > 0
    g = torch.Generator().manual_seed(M + N + K)
    a = (torch.randn(M, K, generator=g) * 0.1).to(torch.bfloat16)
    b = (torch.randn(N, K, generator=g) * 0.1).to(torch.bfloat16)
    ac, bc = a.cuda(), b.cuda()
    out1 = gemm.gemm(ac, bc, out_dtype=torch.float32)
    out2 = gemm.gemm(ac, bc, out_dtype=torch.float32)
    _check(out1, a.double() @ b.double().t(), K, a, b, torch.float32)
    assert torch.equal(out1, out2)
    out16 = gemm.gemm(ac, bc, alpha=2.0)
    _check(out16, 2.0 * (a.double() @ b.double().t()), K, a, b, torch.bfloat16)


@pytest.mark.parametrize("rows,cols", [(16, 3584), (130, 77), (1, 5), (512, 640)])
def test_transpose16_exact(rows, cols):
    g = torch.Generator().manual_seed(rows + cols)
    t = torch.randn(rows, cols, generator=g).to(torch.bfloat16)
    out = gemm.transpose16(t.cuda())
    assert torch.equal(out.cpu(), t.t().contiguous())
    # into the leading columns of a wider zero buffer (the padded LoRA factor layout)
    buf = torch.zeros(cols, rows + 48, dtype=torch.bfloat16, device="cuda")
    gemm.transpose16(t.cuda(), out=buf)
    assert torch.equal(buf[:, :rows].cpu(), t.t()) and torch.all(buf[:, rows:] == 0)


def test_transposed_frozen_cache_follows_the_weight():
    w = torch.randn(96, 128, device="cuda").to(torch.bfloat16)
    t1 = gemm.transposed_frozen(w)
    assert gemm.transposed_frozen(w) is t1 and torch.equal(t1, w.t())
    w.mul_(2)  # an in-place update bumps the version: the cache must not serve the old one
    t2 = gemm.transposed_frozen(w)
    assert t2 is not t1 and torch.equal(t2, w.t())


@pytest.mark.parametrize("M,N,K,K2", [(4096, 512, 3584, 64), (300, 520, 256, 64),
                                      (256, 384, 128, 128), (64, 3584, 0, 64),
                                      (4096, 4608, 256, 64), (300, 256, 64, 320),
                                      (256, 3584, 128, 1024)])
def test_gemm_nt_cat(M, N, K, K2):
    """a b^T + a2 b2^T over the concatenated K in one GEMM (split-K included for 4096x512; a
    second segment longer than 128 with a first of at most 128 swaps their roles)."""
    print(f"gemm_nt_cat M={M} N={N} K={K} K2={K2}", flush=True)
    g = torch.Generator().manual_seed(M + N + K + K2)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    b = torch.randn(N, K, generator=g).to(torch.bfloat16)
    a2 = torch.randn(M, K2, generator=g).to(torch.bfloat16)
    b2 = torch.randn(N, K2, generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    ref = a.double() @ b.double().t() + a2.double() @ b2.double().t() + bias.double()
    for out_dtype in (torch.bfloat16, torch.float32):
        out = torch.empty(M, N, dtype=out_dtype, device="cuda")
        gemm.gemm_nt_cat(a.cuda(), b.cuda(), a2.cuda(), b2.cuda(), out, bias=bias.cuda())
        amax = max(t.abs().max().item() if t.numel() else 0.0 for t in (a, a2))
        bmax = max(t.abs().max().item() if t.numel() else 0.0 for t in (b, b2))
        bound = 4 * 2.0**-22 * (K + K2) * amax * bmax
        if out_dtype != torch.float32:
            bound = bound + 2.0**-8 * ref.abs()
        assert torch.all((out.double().cpu() - ref).abs() <= bound)


@pytest.mark.parametrize("M,K,out_cols,dtype", [(4096, 3584, 64, torch.bfloat16),
                                                (4096, 18944, 64, torch.bfloat16),
                                                (77, 96, 16, torch.bfloat16),
                                                (1000, 512, 40, torch.bfloat16),
                                                (512, 8192, 64, torch.bfloat16),
                                                (1100, 8192, 40, torch.bfloat16),
                                                (2048, 8192, 64, torch.float16)])
def test_lora_down(M, K, out_cols, dtype):
    """out[:, :16] = alpha x y^T, out[:, 16:] = 0 and the transposed copy equal to out[:, :16]
    bit for bit, with and without the split-K workspace (512 x 8192 splits; 4096 x 18944 and
    1100 x 8192 take 64-row blocks split over K, the latter with row groups past M)."""
    print(f"lora_down M={M} K={K} {dtype}", flush=True)
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    y = (torch.randn(16, K, generator=g) * 0.25).to(dtype)
    ref = 2.0 * (x.double() @ y.double().t())
    out = torch.full((M, out_cols), 3.0, dtype=dtype, device="cuda")
    out_t = gemm.lora_t_buffer(M, dtype, "cuda")
    gemm.lora_down(x.cuda(), y.cuda(), out, alpha=2.0, out_t=out_t)
    rnd = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11  # one rounding to the output
    bound = 2 * 4 * 2.0**-22 * K * x.abs().max().item() * y.abs().max().item() + rnd * ref.abs()
    assert torch.all((out[:, :16].double().cpu() - ref).abs() <= bound)
    assert torch.all(out[:, 16:] == 0)
    assert torch.equal(out_t, out[:, :16].t())


def _pt(M, g):
    """A [16, M] token-contiguous operand with a padded row stride, as lora_down writes it."""
    buf = torch.randn(16, (M + 7) // 8 * 8 + 8, generator=g).to(torch.bfloat16)
    return buf[:, :M]


@pytest.mark.parametrize("M,N", [(4096, 18944), (4096, 3584), (4096, 512), (1000, 3584),
                                 (100, 520), (33, 8)])
def test_lora_wgrad(M, N):
    """fp32 [N, 16] = alpha q^T pt^T (a reduction over the M token rows, split over workgroups
    and summed in split order); ragged M exercises the partial 8-row groups."""
    print(f"lora_wgrad M={M} N={N}", flush=True)
    g = torch.Generator().manual_seed(M * 3 + N)
    q = torch.randn(M, N, generator=g).to(torch.bfloat16)
    pt = _pt(M, g)
    ref = 0.5 * (q.double().t() @ pt.double().t())
    pt_dev = gemm.lora_t_buffer(M, torch.bfloat16, "cuda")  # row stride a multiple of 8
    pt_dev.copy_(pt)
    out = gemm.lora_wgrad(pt_dev, q.cuda(), alpha=0.5)
    assert out.shape == (N, 16) and out.dtype == torch.float32
    bound = 0.5 * 4 * 2.0**-22 * M * q.abs().max().item() * pt.abs().max().item()
    assert torch.all((out.double().cpu() - ref).abs() <= bound)
    assert torch.equal(out, gemm.lora_wgrad(pt_dev, q.cuda(), alpha=0.5))  # deterministic


@pytest.mark.parametrize("M,K,G,out_cols", [(4096, 3584, 3, 64), (1000, 512, 2, 32),
                                            (77, 96, 4, 64), (512, 8192, 3, 48),
                                            (4096, 18944, 2, 64)])
def test_lora_down_slots(M, K, G, out_cols):
    """G adapters in one pass over x: out[:, :16G] = alpha x y^T for y [16G, K], zeros after,
    the transposed copy exact, and each slot bit-identical to a single-adapter call where that
    call takes the same 16-row blocks and K splits (the same chunks then reach the same
    accumulator in the same order; a long single-adapter reduction, K >= 8192 with M >= 1024,
    takes 64-row blocks split over K instead)."""
    print(f"lora_down slots={G} M={M} K={K}", flush=True)
    g = torch.Generator().manual_seed(M + K + G)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    y = (torch.randn(16 * G, K, generator=g) * 0.25).to(torch.bfloat16)
    ref = 2.0 * (x.double() @ y.double().t())
    xd, yd = x.cuda(), y.cuda()
    out = torch.full((M, out_cols), 3.0, dtype=torch.bfloat16, device="cuda")
    out_t = gemm.lora_t_buffer(M, torch.bfloat16, "cuda", rows=16 * G)
    gemm.lora_down(xd, yd, out, alpha=2.0, out_t=out_t)
    bound = 2 * 4 * 2.0**-22 * K * x.abs().max().item() * y.abs().max().item() + 2.0**-8 * ref.abs()
    assert torch.all((out[:, :16 * G].double().cpu() - ref).abs() <= bound)
    assert torch.all(out[:, 16 * G:] == 0)
    assert torch.equal(out_t, out[:, :16 * G].t())
    same_path = K < 8192 or M < 1024
    for s in range(G):
        one = torch.empty((M, 16), dtype=torch.bfloat16, device="cuda")
        gemm.lora_down(xd, yd[16 * s:16 * s + 16].contiguous(), one, alpha=2.0)
        if same_path:
            assert torch.equal(one, out[:, 16 * s:16 * s + 16]), s
        else:
            assert torch.all((one.double().cpu() - ref[:, 16 * s:16 * s + 16]).abs()
                             <= bound[:, 16 * s:16 * s + 16]), s


@pytest.mark.parametrize("M,N,G", [(4096, 3584, 3), (4096, 3584, 2), (100, 520, 2),
                                   (1000, 3584, 4), (33, 8, 3), (4096, 18944, 2)])
def test_lora_wgrad_slots(M, N, G):
    """G adapters' gradients in one pass over q: fp32 [N, 16G] = alpha q^T pt^T for pt
    [16G, M], and its transposed form exact."""
    print(f"lora_wgrad slots={G} M={M} N={N}", flush=True)
    g = torch.Generator().manual_seed(M * 5 + N + G)
    q = torch.randn(M, N, generator=g).to(torch.bfloat16)
    pt = torch.randn(16 * G, M, generator=g).to(torch.bfloat16)
    ref = 0.5 * (q.double().t() @ pt.double().t())
    pt_dev = gemm.lora_t_buffer(M, torch.bfloat16, "cuda", rows=16 * G)
    pt_dev.copy_(pt)
    qd = q.cuda()
    out = gemm.lora_wgrad(pt_dev, qd, alpha=0.5)
    assert out.shape == (N, 16 * G) and out.dtype == torch.float32
    bound = 0.5 * 4 * 2.0**-22 * M * q.abs().max().item() * pt.abs().max().item()
    assert torch.all((out.double().cpu() - ref).abs() <= bound)
    assert torch.equal(gemm.lora_wgrad(pt_dev, qd, alpha=0.5, transposed=True), out.t())


@pytest.mark.parametrize("pad", [64, 24, 20])  # 16-B chunks per item; 20: the per-row form
@pytest.mark.parametrize("K,N", [(3584, 512), (256, 18944), (18944, 3584), (8, 8)])
def test_lora_pack_is_exact(K, N, pad):
    """The packed adapter operands equal torch's own casts of A, A^T, s*B and B^T (RNE)."""
    print(f"lora_pack K={K} N={N} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(K + N)
    a = torch.randn(16, K, generator=g) * 0.25
    b = torch.randn(N, 16, generator=g) * 0.01
    for dt in (torch.bfloat16, torch.float16):
        a16, at, bs, bt = gemm.lora_pack(a.cuda(), b.cuda(), 2.0, dt, pad=pad)
        assert torch.equal(a16.cpu(), a.to(dt))
        assert torch.equal(at[:, :16].cpu(), a.t().to(dt)) and torch.all(at[:, 16:] == 0)
        assert torch.equal(bs[:, :16].cpu(), (2.0 * b).to(dt)) and torch.all(bs[:, 16:] == 0)
        assert torch.equal(bt.cpu(), b.t().to(dt))


@pytest.mark.parametrize("M,N", [(4096, 3584), (100, 520)])
def test_lora_wgrad_transposed_output(M, N):
    g = torch.Generator().manual_seed(N)
    q = torch.randn(M, N, generator=g).to(torch.bfloat16).cuda()
    pt = gemm.lora_t_buffer(M, torch.bfloat16, "cuda")
    pt.copy_(torch.randn(16, M, generator=g).to(torch.bfloat16))
    assert torch.equal(gemm.lora_wgrad(pt, q, transposed=True), gemm.lora_wgrad(pt, q).t())
