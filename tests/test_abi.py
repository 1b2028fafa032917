"""The C-ABI library: it loads, exports every symbol include/*.h declares, the ctypes binding
covers exactly those, and argument checks return status codes without launching anything
(so these run without a GPU)."""

import ctypes
import re
from pathlib import Path

import pytest

from hackathon_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def _no_device():
    """The fake-pointer calls below are only safe where no GPU is visible: a call that passed
    its checks by mistake would launch on a bad address. (Counting devices does not initialise
    the GPU.)"""
    import torch

    return torch.cuda.device_count() == 0


needs_no_device = pytest.mark.skipif(not _no_device(),
                                     reason="fake-pointer argument checks run only without a GPU")


@pytest.fixture(scope="session")
def lib():
    if not _lib.LIB_PATH.exists():
        from hackathon_amd import build

        build.build()
    return _lib.load()


def header_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(qlora_\w+)\s*\(", text))
    return names


def test_header_declares_the_kernel_set():
    syms = header_symbols()
    for name in ("qlora_nf4_dequant", "qlora_rmsnorm_fwd", "qlora_rmsnorm_bwd", "qlora_rope_qk",
                 "qlora_swiglu_fwd", "qlora_swiglu_bwd", "qlora_lora_dropout_scale",
                 "qlora_lora_scaled_add", "qlora_ce_rows", "qlora_gemm"):
        assert name in syms


def test_library_exports_every_declared_symbol(lib):
    missing = [s for s in sorted(header_symbols()) if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_covers_exactly_the_header():
    assert set(_lib.exported_symbols()) == header_symbols()


def test_version_and_error_text(lib):
    assert lib.qlora_abi_version() == _lib.ABI_VERSION
    assert lib.qlora_strerror(0) == b"ok"
    assert b"dtype" in lib.qlora_strerror(-2)


@needs_no_device
def test_rejected_arguments_return_codes(lib):
    P = ctypes.c_void_p
    fake = P(0x1000)  # never dereferenced: every call below is rejected before any launch
    # odd weight count
    assert lib.qlora_nf4_dequant(fake, 3, fake, 1, fake, fake, 0.0, 64, 256, fake, fake, 2,
                                 None) == -1
    # nested without a code map
    assert lib.qlora_nf4_dequant(fake, 64, fake, 1, None, fake, 0.0, 64, 256, fake, fake, 2,
                                 None) == -1
    # odd blocksize
    assert lib.qlora_nf4_dequant(fake, 64, fake, 0, None, None, 0.0, 63, 1, fake, fake, 2,
                                 None) == -1
    # unknown output dtype
    assert lib.qlora_nf4_dequant(fake, 64, fake, 0, None, None, 0.0, 64, 1, fake, fake, 7,
                                 None) == -2
    # grouped dequant: empty or oversized group, a weight the vector path cannot take, a
    # 32-bit transposed output, a misaligned output block
    W = _lib.Nf4Weight
    one = (W * 1)(W(0x1000, 64, 64, 0x1000, 0x1000, 0x1000, 0.0, 64, 256, 0x1000))
    assert lib.qlora_nf4_dequant_group(one, 0, 1, fake, 2, None) == -1
    assert lib.qlora_nf4_dequant_group((W * 5)(*([one[0]] * 5)), 5, 1, fake, 2, None) == -1
    assert lib.qlora_nf4_dequant_group(one, 1, 1, None, 2, None) == -1
    assert lib.qlora_nf4_dequant_group((W * 1)(W(0x1000, 3, 6, 0x1000, 0x1000, 0x1000, 0.0, 64,
                                                 256, 0x1000)), 1, 1, fake, 2, None) == -4
    assert lib.qlora_nf4_dequant_group((W * 1)(W(0x1000, 64, 64, 0x1000, 0x1000, 0x1000, 0.0, 6,
                                                 256, 0x1000)), 1, 1, fake, 2, None) == -1
    assert lib.qlora_nf4_dequant_group((W * 1)(W(0x1000, 64, 64, 0x1000, None, 0x1000, 0.0, 64,
                                                 256, 0x1000)), 1, 1, fake, 2, None) == -1
    assert lib.qlora_nf4_dequant_group(one, 1, 1, fake, 7, None) == -2
    t_one = (W * 1)(W(0x1000, 64, 128, 0x1000, 0x1000, 0x1000, 0.0, 64, 256, 0x1000))
    assert lib.qlora_nf4_dequant_t_group(t_one, 1, 1, fake, 64, 0, None) == -2
    assert lib.qlora_nf4_dequant_t_group(t_one, 1, 1, fake, 60, 2, None) == -4
    assert lib.qlora_nf4_dequant_t_group(t_one, 1, 1, fake, 8, 2, None) == -1  # ld_out < rows
    assert lib.qlora_nf4_dequant_t_group((W * 1)(W(0x1000, 64, 96, 0x1000, 0x1000, 0x1000, 0.0,
                                                   64, 256, 0x1000)), 1, 1, fake, 64, 2,
                                         None) == -4
    assert lib.qlora_nf4_dequant_t_group((W * 1)(W(0x1000, 64, 128, 0x1000, 0x1000, 0x1000, 0.0,
                                                   64, 256, 0x1008)), 1, 1, fake, 64, 2,
                                         None) == -3
    # diagonal weight gradient: offsets not ending at N, no workspace, bad dtype
    offs = _lib.i64_array((0, 64, 128))
    al = (ctypes.c_float * 2)(1.0, 1.0)
    assert lib.qlora_lora_wgrad_diag(fake, 64, fake, 256, 64, 256, 2, 2, offs, al, fake, fake,
                                     1 << 20, None) == -4
    offs = _lib.i64_array((0, 64, 256))
    assert lib.qlora_lora_wgrad_diag(fake, 64, fake, 256, 64, 256, 2, 2, offs, al, fake, None,
                                     1 << 20, None) == -1
    assert lib.qlora_lora_wgrad_diag(fake, 64, fake, 256, 64, 256, 2, 0, offs, al, fake, fake,
                                     1 << 20, None) == -2
    assert lib.qlora_lora_wgrad_diag(fake, 64, fake, 256, 64, 256, 2, 2, offs, al, fake, fake,
                                     16, None) == -1  # workspace too small
    assert lib.qlora_lora_wgrad_diag_workspace_size(64, 256, 5) == 0
    # rmsnorm: bad dtype, zero columns
    assert lib.qlora_rmsnorm_fwd(fake, 9, 8, fake, 2, fake, 2, 8, fake, 4, 8, 1e-6, None) == -2
    assert lib.qlora_rmsnorm_fwd(fake, 2, 8, fake, 2, fake, 2, 8, fake, 4, 0, 1e-6, None) == -1
    # rope: odd head dim, output dtype not the promotion of the inputs
    s3 = _lib.i64_array((0, 0, 0))
    assert lib.qlora_rope_qk(fake, fake, fake, fake, fake, fake, 2, 2, 2, 1, 1, 1, 1, 7, s3, s3,
                             s3, s3, 0, 0, 0, None) == -1
    assert lib.qlora_rope_qk(fake, fake, fake, fake, fake, fake, 2, 2, 0, 1, 1, 1, 1, 8, s3, s3,
                             s3, s3, 0, 0, 0, None) == -2
    # swiglu: negative size
    assert lib.qlora_swiglu_fwd(fake, fake, fake, 2, -1, None) == -1
    # scaled add: output dtype must be promote(base, lo)
    assert lib.qlora_lora_scaled_add(fake, 0, 8, fake, 1, 8, fake, 1, 8, 2, 8, 2.0, None) == -2
    # ce_rows: unknown ignore mode
    assert lib.qlora_ce_rows(fake, 2, 8, 2, 8, fake, fake, fake, None, None, 2, 0, 1.0,
                             None) == -1
    # pack jobs: negative count, a pad below one slot, no descriptors, a misaligned output
    # base, an fp32 output; no jobs is a no-op
    assert lib.qlora_lora_pack_jobs(fake, -1, 8, fake, 2, 64, None) == -1
    assert lib.qlora_lora_pack_jobs(fake, 1, 8, fake, 2, 12, None) == -1
    assert lib.qlora_lora_pack_jobs(None, 1, 8, fake, 2, 64, None) == -1
    assert lib.qlora_lora_pack_jobs(fake, 1, 8, P(0x1008), 2, 64, None) == -3
    assert lib.qlora_lora_pack_jobs(fake, 1, 8, fake, 0, 64, None) == -2
    assert lib.qlora_lora_pack_jobs(None, 0, 0, None, 2, 64, None) == 0
    # ce_rows with the scale in device memory: a gradient asked for without the scale
    assert lib.qlora_ce_rows_scale_ptr(fake, 2, 8, 2, 8, fake, fake, fake, None, None, 1, 1,
                                       None, None) == -1
    # gemm: fp32 inputs are not a matrix-core type; an operand not element-aligned; a leading
    # dimension shorter than the row
    assert lib.qlora_gemm(0, 0, 4, 4, 8, fake, 8, fake, 8, 0, fake, 4, 0, None, 1.0, 0.0,
                          None) == -2
    assert lib.qlora_gemm(0, 0, 4, 4, 8, P(0x1001), 8, fake, 8, 2, fake, 4, 0, None, 1.0, 0.0,
                          None) == -3
    assert lib.qlora_gemm(0, 0, 4, 4, 12, fake, 8, fake, 16, 2, fake, 4, 0, None, 1.0, 0.0,
                          None) == -4
    # cat gemm: the two K segments may not both exceed 128 (the short one is loaded up front)
    assert lib.qlora_gemm_nt_cat(256, 256, 256, fake, 256, fake, 256, 192, fake, 192, fake, 192,
                                 2, fake, 256, 2, None, 1.0, None, 0, None) == -4
    # cat gemm with a residual: none given; an fp32 output; a misaligned residual; a residual
    # row shorter than N; a residual overlapping the output
    other = P(0x100000)
    args = (256, 256, 256, fake, 256, fake, 256, 0, None, 0, None, 0, 2)
    assert lib.qlora_gemm_nt_cat_residual(*args, fake, 256, 2, None, 256, None, 0, None) == -1
    assert lib.qlora_gemm_nt_cat_residual(*args, fake, 256, 0, other, 256, None, 0, None) == -2
    assert lib.qlora_gemm_nt_cat_residual(*args, fake, 256, 2, P(0x100008), 256, None, 0,
                                          None) == -3
    assert lib.qlora_gemm_nt_cat_residual(*args, fake, 256, 2, other, 128, None, 0, None) == -4
    assert lib.qlora_gemm_nt_cat_residual(*args, fake, 256, 2, P(0x1000 + 512), 256, None, 0,
                                          None) == -1
    # rank-16 LoRA kernels: 1 to 4 adapters per call; the workspace query is 0 outside that
    assert lib.qlora_lora_down(fake, 64, fake, 64, 16, 64, 0, 2, fake, 64, 64, 2, 1.0, None, 0,
                               None, 0, None) == -1
    assert lib.qlora_lora_down(fake, 64, fake, 64, 16, 64, 5, 2, fake, 64, 64, 2, 1.0, None, 0,
                               None, 0, None) == -1
    # ... the output must hold the 16 G adapter columns
    assert lib.qlora_lora_down(fake, 64, fake, 64, 16, 64, 3, 2, fake, 64, 32, 2, 1.0, None, 0,
                               None, 0, None) == -1
    assert lib.qlora_lora_wgrad(fake, 64, fake, 64, 64, 64, 5, 2, fake, 0, 1.0, None, 0,
                                None) == -1
    # lane byte offsets are 32-bit: a 64-row block (one adapter, K >= 8192, M >= 1024) spans
    # 128 * ldx bytes, so ldx = 2^24 is refused there; 16-row blocks refuse ldx >= 2^26
    big = 1 << 24
    assert lib.qlora_lora_down(fake, big, fake, 8192, 1024, 8192, 1, 2, fake, 64, 64, 2, 1.0,
                               None, 0, None, 0, None) == -1
    assert lib.qlora_lora_down(fake, 1 << 26, fake, 64, 16, 64, 1, 2, fake, 64, 64, 2,
                               1.0, None, 0, None, 0, None) == -1
    assert lib.qlora_lora_down_workspace_size(4096, 3584, 0) == 0
    assert lib.qlora_lora_wgrad_workspace_size(4096, 3584, 5) == 0
    # fused SwiGLU backward + down-projections: columns a multiple of 32, room for both
    # adapters' 32 output columns, 16-bit dtypes only
    assert lib.qlora_swiglu_bwd_lora_down(fake, 48, fake, 96, fake, 96, fake, 96, fake, 96, 16, 48,
                                          fake, fake, 96, 1.0, 1.0, 2, fake, 64, 64, None, 0,
                                          None, 0, None) == -1
    assert lib.qlora_swiglu_bwd_lora_down(fake, 64, fake, 128, fake, 128, fake, 128, fake, 128, 16,
                                          64, fake, fake, 128, 1.0, 1.0, 2, fake, 64, 16, None, 0,
                                          None, 0, None) == -1
    gr, ga, up, dg, du = (P(0x10000 * (i + 1)) for i in range(5))  # disjoint fake matrices
    assert lib.qlora_swiglu_bwd_lora_down(gr, 64, ga, 128, up, 128, dg, 128, du, 128, 16,
                                          64, fake, fake, 128, 1.0, 1.0, 0, fake, 64, 64, None, 0,
                                          None, 0, None) == -2
    # ... and never in place: an output whose bytes meet an input's is refused before launching
    for dgate, dup in ((ga, du), (dg, up), (dg, gr), (P(0x20000 + 64), du)):
        assert lib.qlora_swiglu_bwd_lora_down(gr, 64, ga, 128, up, 128, dgate, 128, dup, 128,
                                              16, 64, fake, fake, 128, 1.0, 1.0, 2, fake, 64, 64,
                                              None, 0, None, 0, None) == -1
    # ... and with both lora_B gradients: the workspace is required, and neither output may
    # meet an input
    for with_da in (0, 1):  # at least the du partials of the 74 blocks of 256 columns
        assert lib.qlora_swiglu_bwd_lora_workspace_size(4096, 18944, with_da) > 74 * 4096 * 128
    assert lib.qlora_swiglu_bwd_lora_workspace_size(4096, 100, 0) == 0  # cols % 32
    assert lib.qlora_swiglu_bwd_lora(gr, 64, ga, 128, up, 128, dg, 128, du, 128, 16, 64, fake,
                                     fake, 128, fake, fake, 16, 1.0, 1.0, 1.0, 1.0, 2, fake, 64,
                                     64, None, 0, fake, fake, None, 1.0, None, None, 0,
                                     None) == -1
    assert lib.qlora_swiglu_bwd_lora(gr, 64, ga, 128, up, 128, ga, 128, du, 128, 16, 64, fake,
                                     fake, 128, fake, fake, 16, 1.0, 1.0, 1.0, 1.0, 2, fake, 64,
                                     64, None, 0, fake, fake, None, 1.0, None, fake, 1 << 20,
                                     None) == -1
    # ... the down adapter's du^T and dA come together or not at all
    assert lib.qlora_swiglu_bwd_lora(gr, 64, ga, 128, up, 128, dg, 128, du, 128, 16, 64, fake,
                                     fake, 128, fake, fake, 16, 1.0, 1.0, 1.0, 1.0, 2, fake, 64,
                                     64, None, 0, fake, fake, fake, 1.0, None, fake, 1 << 20,
                                     None) == -1
    # SwiGLU forward + the down adapter's u: columns a multiple of 32, never in place
    assert lib.qlora_swiglu_fwd_lora_down(ga, 128, up, 128, dg, 128, 16, 48, fake, 48, 1.0, 2,
                                          fake, 64, 64, None, 0, None, 0, None) == -1
    assert lib.qlora_swiglu_fwd_lora_down(ga, 128, up, 128, up, 128, 16, 64, fake, 64, 1.0, 2,
                                          fake, 64, 64, None, 0, None, 0, None) == -1
    # adamw: a table is required when there is work; the bias correction must be positive
    assert lib.qlora_adamw_fp32(None, 1, 1, 1.0, 0.999, 0.1, 0.001, 1e-3, 1.0, 1e-8, None) == -1
    assert lib.qlora_adamw_fp32(fake, 1, 1, 1.0, 0.999, 0.1, 0.001, 1e-3, 0.0, 1e-8, None) == -1
    assert lib.qlora_adamw_chunk_elems() == 2048
    # add + rmsnorm: the row length must be a multiple of 8; rows must be 16-B aligned
    assert lib.qlora_add_rmsnorm_fwd(fake, fake, 2, 12, 12, fake, 2, fake, 12, fake, 2, 12, fake,
                                     4, 12, 1e-6, None) == -4
    assert lib.qlora_add_rmsnorm_fwd(P(0x1008), fake, 2, 16, 16, fake, 2, fake, 16, fake, 2, 16,
                                     fake, 4, 16, 1e-6, None) == -3
    assert lib.qlora_rmsnorm_bwd_residual(fake, 2, 16, fake, 2, 16, fake, 2, fake, None, 16, fake,
                                          16, 4, 16, None) == -1
    # attention: head_dim must be 128
    strides = (ctypes.c_int64 * 3)(0, 0, 0)
    assert lib.qlora_attn_fwd(fake, fake, fake, fake, None, 2, 1, 1, 1, 64, 64, strides, strides,
                              strides, strides, 0.1, None) == -4


def test_empty_problems_are_no_ops(lib):
    # zero-sized work returns OK without touching the (null) pointers or the device
    assert lib.qlora_nf4_dequant(None, 0, None, 0, None, None, 0.0, 64, 1, None, None, 2,
                                 None) == 0
    assert lib.qlora_swiglu_fwd(None, None, None, 2, 0, None) == 0
    assert lib.qlora_gemm(0, 0, 0, 4, 8, None, 8, None, 8, 2, None, 4, 2, None, 1.0, 0.0,
                          None) == 0


@needs_no_device
def test_noalloc_wgrad_rejects_scratch_beyond_its_array(lib):
    """qlora_lora_wgrad_noalloc returns QL_ESHAPE, launching nothing, when the split partials
    would need more than its 16 MiB array (4 slots, N = 16392, M = 4096: 4 splits x 16392 x 64
    fp32 = 16.8 MB); bad arguments are rejected as by qlora_lora_wgrad."""
    P = ctypes.c_void_p
    fake = P(0x1000)  # never dereferenced: every call below is rejected before any launch
    assert lib.qlora_lora_wgrad_workspace_size(4096, 16392, 4) > 16 << 20
    assert lib.qlora_lora_wgrad_noalloc(fake, 4096, fake, 16392, 4096, 16392, 4, 2, fake, 0,
                                        1.0, None) == -4
    assert lib.qlora_lora_wgrad_noalloc(fake, 4096, fake, 16392, 4096, 16392, 5, 2, fake, 0,
                                        1.0, None) == -1  # slots > 4
    assert lib.qlora_lora_wgrad_noalloc(None, 4096, fake, 512, 4096, 512, 1, 2, fake, 0,
                                        1.0, None) == -1  # null operand
    assert lib.qlora_lora_wgrad_noalloc(fake, 4096, fake, 512, -1, 512, 1, 2, fake, 0,
                                        1.0, None) == -1  # negative size


def test_dropout_keep_threshold_is_the_float_test(lib):
    """The kernels keep an element when its folded Philox word x is >= the threshold; the
    reference keeps it when (float)x * 4.6566127342e-10f > p. The two agree on every word: the
    float test is monotone in x, so checking the words around the threshold, the ends of the
    range and a spread of others pins it (numpy's int32 -> float32 conversion and float32
    product round as the reference's do)."""
    import numpy as np

    from oracle import philox

    rng = np.random.default_rng(7)
    spread = np.concatenate([rng.integers(0, 1 << 31, 200_000, dtype=np.int64),
                             np.arange(0, 1 << 31, (1 << 31) // 4096, dtype=np.int64),
                             np.array([0, 1, (1 << 31) - 1], dtype=np.int64)])
    ps = [0.05, 0.1, 0.2, 0.5, 0.75, 0.9, 1e-9, 0.0, 0.99999994, 1.0, 1.5, -0.25, float("nan"),
          float(np.nextafter(np.float32(0.05), np.float32(1)))]
    for p in ps:
        t = int(lib.qlora_dropout_keep_threshold(ctypes.c_float(p)))
        assert 0 <= t <= 1 << 31
        x = np.concatenate([spread, np.arange(t - 3, t + 4, dtype=np.int64)])
        x = x[(x >= 0) & (x < 1 << 31)]
        u = x.astype(np.int32).astype(np.float32) * philox.SCALE
        want = u > np.float32(p)
        assert np.array_equal(x >= t, want), p
    # the mask's own rate: at p = 0.05 the threshold sits at 5% of the range
    assert abs(int(lib.qlora_dropout_keep_threshold(0.05)) / 2**31 - 0.05) < 1e-6


@needs_no_device
def test_dropout_down_rejects_bad_arguments(lib):
    """qlora_lora_dropout_down returns status codes before any launch: slots outside 1..4 and p
    outside (0, 1) are QL_EINVAL, K not a multiple of 64 or a short stride QL_ESHAPE, a
    misaligned row stride QL_EALIGN."""
    P = ctypes.c_void_p
    fake = P(0x1000)
    seeds = (ctypes.c_uint64 * 4)(1, 2, 3, 4)
    ptrs = (ctypes.c_void_p * 4)(0x1000, 0x2000, 0x3000, 0x4000)

    def call(M=16, K=128, slots=1, p=0.05, ldx=128, u_cols=64, xd_rs=128):
        return lib.qlora_lora_dropout_down(fake, ldx, fake, 128, M, K, slots, 2, seeds, p,
                                           1.0 / (1.0 - p) if p < 1 else 1.0, ptrs, xd_rs, ptrs,
                                           K, fake, 64, u_cols, None, 0, None, 0, None)

    assert call(slots=0) == -1 and call(slots=5) == -1
    assert call(p=0.0) == -1 and call(p=1.0) == -1
    assert call(K=96, ldx=96, xd_rs=96) == -4
    assert call(ldx=64) == -4 and call(u_cols=16 * 1 - 8) == -4
    assert call(ldx=132) == -3
    assert call(M=0) == 0


@needs_no_device
def test_wgrad_masked_rejects_bad_arguments(lib):
    """qlora_lora_wgrad_masked: a null or misaligned keep-bit pointer, a group stride below N or
    not a multiple of 8 are rejected before any launch."""
    P = ctypes.c_void_p
    fake = P(0x1000)
    ok = (ctypes.c_void_p * 2)(0x1000, 0x2000)
    bad = (ctypes.c_void_p * 2)(0x1000, 0x2004)
    null = (ctypes.c_void_p * 2)(0x1000, 0)

    def call(bits=ok, gs=512, N=512, slots=2):
        return lib.qlora_lora_wgrad_masked(fake, 64, fake, 512, 64, N, slots, 2, bits, gs,
                                           1.0 / 0.95, fake, 1.0, None, 0, None)

    assert call(bits=null) == -1 and call(slots=5) == -1
    assert call(bits=bad) == -3
    assert call(gs=504) == -4 and call(gs=516) == -4 and call(N=500, gs=512) == -4
