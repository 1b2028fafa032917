"""The 4-bit base GEMM with the NF4 weight dequantised inside the GEMM (qlora_gemm_nf4)
against the dense GEMM on the weight qlora_nf4_dequant writes (qlora_gemm_nt_cat): the same
16-bit weight values and the same per-element K order, so the outputs must be identical bit
for bit. The first cases are also checked against an fp64 product to the fp32 accumulation
bound, which pins both GEMMs independently of each other."""

import pytest
import torch

from hackathon_amd import gemm, nf4, quant

pytestmark = pytest.mark.gpu

CASES = [
    # M, N, K, nested, dtype, blocksize, LoRA segment
    (4096, 18944, 3584, True, torch.bfloat16, 64, True),    # Qwen2.5-7B gate/up projection
    (4096, 3584, 18944, True, torch.bfloat16, 64, False),   # Qwen2.5-7B down projection
    (512, 512, 4096, True, torch.bfloat16, 64, True),       # few tiles: split over K
    (300, 520, 1024, False, torch.float16, 128, True),      # ragged M and N, plain absmax
    (64, 3584, 3584, True, torch.bfloat16, 256, False),     # one M tile
    (1000, 264, 64 * 3, True, torch.float16, 64, False),    # 3 K steps, N not a multiple of 8
]


def _weights(N, K, nested, blocksize, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(N, K, device="cuda", generator=g) * 0.02
    return quant.quantize_nf4(w, blocksize, compress_statistics=nested)


@pytest.mark.parametrize("M,N,K,nested,dtype,bs,lora", CASES)
def test_gemm_nf4_matches_the_dense_gemm_on_the_dequantised_weight(M, N, K, nested, dtype, bs,
                                                                    lora):
    print(f"gemm_nf4 M={M} N={N} K={K} nested={nested} {dtype} bs={bs} lora={lora}", flush=True)
    packed, st = _weights(N, K, nested, bs, seed=M + N)
    g = torch.Generator(device="cuda").manual_seed(K)
    x = torch.randn(M, K, device="cuda", generator=g).to(dtype)
    bias = (torch.randn(N, device="cuda", generator=g) * 0.1).to(dtype)
    a2 = b2 = None
    if lora:
        a2 = torch.zeros(M, 64, device="cuda", dtype=dtype)
        a2[:, :16] = torch.randn(M, 16, device="cuda", generator=g).to(dtype)
        b2 = torch.zeros(N, 64, device="cuda", dtype=dtype)
        b2[:, :16] = (torch.randn(N, 16, device="cuda", generator=g) * 0.02).to(dtype)
    assert nf4.fused_gemm_ok(st, packed, x)
    w = nf4.dequantize_nf4(packed, st, dtype)
    want = torch.empty(M, N, device="cuda", dtype=dtype)
    gemm.gemm_nt_cat(x, w, a2, b2, want, bias=bias, alpha=0.5)
    got = nf4.gemm_nf4(x, packed, st, a2=a2, b2=b2, bias=bias, alpha=0.5)
    torch.cuda.synchronize()
    assert torch.equal(got, want), (got.float() - want.float()).abs().max().item()
    if M * N * K <= 4096 * 18944 * 3584 and (M, N) != (300, 520):
        ref = x.double() @ w.double().t()
        mag = x.double().abs() @ w.double().abs().t()
        if lora:
            ref += a2.double() @ b2.double().t()
            mag += a2.double().abs() @ b2.double().abs().t()
        ref = 0.5 * ref + bias.double()
        # fp32 accumulation over K (+ K2) terms, then one rounding to the 16-bit output
        ulp16 = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
        bound = (K + 64) * 2.0 ** -24 * 0.5 * mag + ulp16 * ref.abs() + 1e-6
        assert torch.all((got.double() - ref).abs() <= bound)


def test_gemm_nf4_refuses_what_it_cannot_take():
    packed, st = _weights(256, 96, True, 32, seed=1)  # K not a multiple of 64, blocksize 32
    x = torch.zeros(8, 96, device="cuda", dtype=torch.bfloat16)
    assert not nf4.fused_gemm_ok(st, packed, x)
    with pytest.raises(RuntimeError):
        nf4.gemm_nf4(x, packed, st)


def test_small_batch_forward_takes_the_fused_gemm_with_identical_results(monkeypatch):
    """At 128 tokens every 4-bit projection of a Qwen2.5-7B-shaped layer (the q/k/v and
    gate/up groups, o and down alone) runs gemm_nf4; loss and adapter gradients are identical
    bit for bit to the dequantise-then-GEMM path the same model takes at any row count."""
    from hackathon_amd import qlora_step

    cfg = qlora_step.qwen2_config(num_hidden_layers=1, vocab_size=2048)
    model = qlora_step.build_qlora_model(cfg, "cuda", seed=3)
    qlora_step.patched_mode()
    ids, labels = qlora_step.make_batch(1, 128, cfg.vocab_size)
    calls = []
    real = nf4.gemm_nf4

    def counted(*a, **k):
        calls.append(a[2].shape)
        return real(*a, **k)
    monkeypatch.setattr(nf4, "gemm_nf4", counted)

    def run():
        model.zero_grad(set_to_none=True)
        loss = qlora_step.QLoRAStep(model, fused_head=True).forward_backward(ids, labels)
        return loss, [p.grad.clone() for p in qlora_step.lora_parameters(model)]
    loss_f, grads_f = run()
    assert len(calls) == 7  # q, k, v, o, gate, up, down
    monkeypatch.setattr(nf4, "FUSED_GEMM_MAX_ROWS", 0)
    calls.clear()
    loss_d, grads_d = run()
    assert not calls
    assert torch.equal(loss_f, loss_d)
    assert all(torch.equal(a, b) for a, b in zip(grads_f, grads_d))
