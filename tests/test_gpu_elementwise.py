"""RMSNorm, RoPE, SwiGLU and the LoRA cast/add kernels on the GPU vs the CPU oracle.

Tolerances: bf16 outputs within rtol = atol = 1e-2 (the kernel set's bf16 bar); fp16 and
fp32 within the reference's TOL (solution/_testing.py:12); the dropout mask bit-exact.
"""

import numpy as np
import pytest
import torch

from hackathon_amd import lora, rmsnorm, rope, swiglu
from oracle import ops, philox
from tests._util import BF16_TOL, TOL

pytestmark = pytest.mark.gpu


def tol(dtype):
    return BF16_TOL if dtype == torch.bfloat16 else dict(rtol=TOL[dtype] * 2, atol=TOL[dtype] * 2)


# ---- RMSNorm ------------------------------------------------------------------------------------
@pytest.mark.parametrize("shape,x_dtype,w_dtype", [
    ((4, 2048, 1536), torch.bfloat16, torch.bfloat16),   # Qwen2.5-1.5B, batch 4 x seq 2048
    ((2, 8, 3584), torch.bfloat16, torch.bfloat16),      # Qwen2.5-7B hidden
    ((2, 5, 1536), torch.float32, torch.float32),
    ((2, 5, 1536), torch.float16, torch.float32),
    ((3, 7, 1000), torch.bfloat16, torch.float32),
    ((3, 7, 1003), torch.bfloat16, torch.bfloat16),      # row not a multiple of 8: generic path
    ((1, 3, 8192), torch.bfloat16, torch.bfloat16),      # longest fast-path row
    ((1, 2, 9000), torch.float32, torch.float32),        # longer rows: generic path
])
def test_rmsnorm_fwd_bwd(shape, x_dtype, w_dtype):
    print(f"rmsnorm {shape} {x_dtype} {w_dtype}", flush=True)
    g = torch.Generator().manual_seed(0)
    H = shape[-1]
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(w_dtype)
    x = torch.randn(shape, generator=g).to(x_dtype)
    y_ref, rstd_ref = ops.rmsnorm_fwd(x, w, 1e-6)
    xg = x.cuda().requires_grad_()
    y = rmsnorm.rmsnorm(xg, w.cuda(), 1e-6)
    assert y.dtype == y_ref.dtype and y.shape == y_ref.shape
    # y = w * round_{x dtype}(x * r): a 16-bit x bounds the precision of y whatever its dtype
    # (the reference's test uses TOL[x_dtype], solution/test_rmsnorm.py:36)
    y_tol = tol(x_dtype) if x_dtype != torch.float32 else tol(y.dtype)
    torch.testing.assert_close(y.cpu().float(), y_ref.float(), **y_tol)
    dy = torch.randn(shape, generator=g).to(y.dtype)
    y.backward(dy.cuda())
    dx_ref = ops.rmsnorm_bwd(dy, x, w, rstd_ref)
    assert xg.grad.dtype == x.dtype
    torch.testing.assert_close(xg.grad.cpu().float(), dx_ref.float(), **tol(x.dtype))


def test_rmsnorm_noncontiguous_rows():
    print("rmsnorm strided rows", flush=True)
    g = torch.Generator().manual_seed(1)
    base = torch.randn(6, 2 * 1536, generator=g).to(torch.bfloat16)
    x = base[:, :1536]                      # row stride 3072
    w = (1 + 0.1 * torch.randn(1536, generator=g)).to(torch.bfloat16)
    y = rmsnorm.rmsnorm(x.cuda(), w.cuda(), 1e-6)
    torch.testing.assert_close(y.cpu().float(), ops.rmsnorm_fwd(x, w, 1e-6)[0].float(), **BF16_TOL)


# ---- RoPE ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("B,S,HQ,HK,dtype,halves_equal,batch_cos", [
    (4, 2048, 12, 2, torch.bfloat16, True, 1),     # Qwen2.5-1.5B attention, positions 0..2047
    (2, 64, 28, 4, torch.bfloat16, True, 2),       # Qwen2.5-7B head layout
    (2, 6, 12, 2, torch.float32, True, 1),
    (2, 6, 12, 2, torch.float16, False, 2),
    (2, 6, 12, 2, torch.float32, False, 1),
])
def test_rope_fwd_bwd(B, S, HQ, HK, dtype, halves_equal, batch_cos):
    print(f"rope B={B} S={S} HQ={HQ} HK={HK} {dtype}", flush=True)
    g = torch.Generator().manual_seed(0)
    D = 128
    q = torch.randn(B, S, HQ, D, generator=g).to(dtype).transpose(1, 2)
    k = torch.randn(B, S, HK, D, generator=g).to(dtype).transpose(1, 2)
    if halves_equal:
        cos, sin = ops.qwen_cos_sin(batch_cos, S, D, dtype=dtype)
    else:
        cos = torch.randn(batch_cos, S, D, generator=g).to(dtype)
        sin = torch.randn(batch_cos, S, D, generator=g).to(dtype)
    qo_ref, ko_ref = ops.rope(q, k, cos, sin)
    qg = q.cuda().requires_grad_()
    kg = k.cuda().requires_grad_()
    qo, ko = rope.HipRoPE.apply(qg, kg, cos.cuda(), sin.cuda())
    t = tol(dtype) if halves_equal else {k_: v * 4 for k_, v in tol(dtype).items()}
    for got, want in ((qo, qo_ref), (ko, ko_ref)):
        assert got.dtype == want.dtype and got.shape == want.shape
        assert got.stride() == (got.shape[2] * got.shape[1] * D, D, got.shape[1] * D, 1)
        torch.testing.assert_close(got.cpu().float(), want.float(), **t)
    gq = torch.randn(qo.shape, generator=g).to(dtype)
    gk = torch.randn(ko.shape, generator=g).to(dtype)
    torch.autograd.backward((qo, ko), (gq.cuda(), gk.cuda()))
    dq_ref, dk_ref = ops.rope(gq, gk, cos, sin, backward=True)
    torch.testing.assert_close(qg.grad.cpu().float(), dq_ref.float(), **t)
    torch.testing.assert_close(kg.grad.cpu().float(), dk_ref.float(), **t)


def test_rope_patch_matches_transformers_on_gpu():
    from transformers.models.qwen2 import modeling_qwen2 as m

    rope.patch()
    assert getattr(m.apply_rotary_pos_emb, "_solution_patch", False)
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 9, 4, 64, generator=g).transpose(1, 2).cuda()
    k = torch.randn(2, 9, 2, 64, generator=g).transpose(1, 2).cuda()
    cos, sin = (t.cuda() for t in ops.qwen_cos_sin(1, 9, 64))
    got = m.apply_rotary_pos_emb(q, k, cos, sin)
    want = m.apply_rotary_pos_emb._original(q, k, cos, sin)
    for a, b in zip(got, want):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


# ---- SwiGLU -------------------------------------------------------------------------------------
@pytest.mark.parametrize("shape,dtype", [
    ((4096, 18944), torch.bfloat16),   # Qwen2.5-7B MLP intermediate, 4096 tokens
    ((3, 77, 1001), torch.bfloat16),
    ((4, 512, 8960), torch.float16),
    ((3, 77, 1001), torch.float32),
])
def test_swiglu_fwd_bwd(shape, dtype):
    print(f"swiglu {shape} {dtype}", flush=True)
    g = torch.Generator().manual_seed(0)
    gate = torch.randn(shape, generator=g).to(dtype)
    up = torch.randn(shape, generator=g).to(dtype)
    grad = torch.randn(shape, generator=g).to(dtype)
    gg, ug = gate.cuda().requires_grad_(), up.cuda().requires_grad_()
    out = swiglu.swiglu(gg, ug)
    torch.testing.assert_close(out.cpu().float(), ops.swiglu_fwd(gate, up).float(), **tol(dtype))
    out.backward(grad.cuda())
    dg_ref, du_ref = ops.swiglu_bwd(grad, gate, up)
    torch.testing.assert_close(gg.grad.cpu().float(), dg_ref.float(), **tol(dtype))
    torch.testing.assert_close(ug.grad.cpu().float(), du_ref.float(), **tol(dtype))


# ---- LoRA dropout/cast and scaled add ----------------------------------------------------------
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_dropout_cast_without_dropout_is_an_exact_cast(out_dtype):
    x = torch.randn(3, 7, 1536, device="cuda", requires_grad=True)
    y = lora.DropoutCast.apply(x, 0.0, 0, out_dtype)
    assert y.dtype == out_dtype
    torch.testing.assert_close(y, x.detach().to(out_dtype), atol=0, rtol=0)
    gr = torch.randn_like(y)
    y.backward(gr)
    assert x.grad.dtype == x.dtype
    torch.testing.assert_close(x.grad, gr.float(), atol=0, rtol=0)


@pytest.mark.parametrize("rows,cols", [(64, 1536), (2048, 1536), (5, 1001)])
def test_dropout_mask_is_the_reference_mask(rows, cols):
    print(f"dropout {rows}x{cols}", flush=True)
    p, seed = 0.05, 1234
    x = torch.randn(rows, cols, device="cuda", requires_grad=True)
    y = lora.DropoutCast.apply(x, p, seed, torch.float32)
    keep = torch.from_numpy(philox.keep_mask(seed, rows, cols, p))
    assert torch.equal((y != 0).cpu(), keep & (x.detach().cpu() != 0))
    torch.testing.assert_close(y.cpu(), ops.dropout_scale(x.detach().cpu(), p, seed,
                                                          1 / (1 - p), torch.float32),
                               rtol=0, atol=0)
    y.backward(torch.ones_like(y))
    torch.testing.assert_close(x.grad.cpu(), keep.float() * np.float32(1 / (1 - p)), rtol=0, atol=0)
    rate = 1 - keep.float().mean().item()
    assert abs(rate - p) < 0.01 + 3 / np.sqrt(rows * cols)


@pytest.mark.parametrize("out_features", [1536, 256, 1001])
def test_scaled_add(out_features):
    g = torch.Generator().manual_seed(0)
    base = torch.randn(2, 5, out_features, generator=g)
    lo = torch.randn(2, 5, out_features, generator=g).to(torch.float16)
    bg, lg = base.cuda().requires_grad_(), lo.cuda().requires_grad_()
    out = lora.ScaledAdd.apply(bg, lg, 2.0)
    assert out.dtype == torch.float32
    torch.testing.assert_close(out.cpu(), ops.scaled_add(base, lo, 2.0), atol=1e-6, rtol=1e-6)
    gr = torch.randn(out.shape, generator=g)
    out.backward(gr.cuda())
    torch.testing.assert_close(bg.grad.cpu(), gr)
    assert lg.grad.dtype == torch.float16
    torch.testing.assert_close(lg.grad.cpu().float(), (gr * 2.0).to(torch.float16).float(),
                               atol=0, rtol=0)
