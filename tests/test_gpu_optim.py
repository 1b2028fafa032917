"""FusedAdamW (one HIP launch over every fp32 adapter tensor) against torch.optim.AdamW on the
same parameters and gradients, over six steps: parameters and both moments within about two
fp32 ulps per step (rtol 2e-6, atol 1e-7 at |p| ~ 0.1). The per-element operations follow
torch's order; whether a*b+c is contracted into one fma can differ from torch's build, a
last-bit difference that compounds over steps. Covers
tensor sizes that are not multiples of the 4-wide vector or of the 2048-element chunk, an
unaligned tensor (scalar path), weight decay, and tensors torch must update itself (bf16)."""

import pytest
import torch

from hackathon_amd.optim import FusedAdamW

pytestmark = pytest.mark.gpu


def _params(seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    big = torch.randn(5003, device="cuda", generator=g)
    shapes = [(16, 3584), (3584, 16), (7,), (2048,), (4099,), (16, 18944)]
    ps = [torch.randn(s, device="cuda", generator=g) * 0.1 for s in shapes]
    ps.append(big[1:4001])  # 4-byte offset: not 16-B aligned
    return ps


@pytest.mark.parametrize("wd", [0.0, 0.01])
def test_fused_adamw_matches_torch(wd):
    print(f"fused adamw wd={wd}", flush=True)
    base = _params(0)
    p_ref = [torch.nn.Parameter(t.clone()) for t in base]
    p_fus = [torch.nn.Parameter(t.clone()) for t in base]
    opt_ref = torch.optim.AdamW(p_ref, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd,
                                foreach=False)
    opt_fus = FusedAdamW(p_fus, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd)
    g = torch.Generator(device="cuda").manual_seed(1)
    for step in range(6):
        for a, b in zip(p_ref, p_fus):
            grad = torch.randn(a.shape, device="cuda", generator=g) * (0.1 + step)
            a.grad = grad.clone()
            b.grad = grad.clone()
        opt_ref.step()
        opt_fus.step()
        for a, b in zip(p_ref, p_fus):
            torch.testing.assert_close(b, a, rtol=2e-6, atol=1e-7)
            sa, sb = opt_ref.state[a], opt_fus.state[b]
            torch.testing.assert_close(sb["exp_avg"], sa["exp_avg"], rtol=2e-6, atol=1e-7)
            torch.testing.assert_close(sb["exp_avg_sq"], sa["exp_avg_sq"], rtol=2e-6, atol=1e-7)
            assert float(sb["step"]) == float(sa["step"]) == step + 1


def test_fused_adamw_grads_set_to_none_and_other_dtypes():
    """Gradients re-created each step (new pointers) and a bf16 parameter (torch's step)."""
    base = _params(2)[:3]
    p_ref = [torch.nn.Parameter(t.clone()) for t in base] + [
        torch.nn.Parameter(torch.randn(33, device="cuda", dtype=torch.bfloat16))]
    p_fus = [torch.nn.Parameter(t.detach().clone()) for t in p_ref]
    opt_ref = torch.optim.AdamW(p_ref, lr=3e-3, weight_decay=0.05, foreach=False)
    opt_fus = FusedAdamW(p_fus, lr=3e-3, weight_decay=0.05)
    for step in range(3):
        for a, b in zip(p_ref, p_fus):
            grad = torch.randn_like(a)
            a.grad, b.grad = grad.clone(), grad.clone()
        opt_ref.step()
        opt_fus.step()
        opt_ref.zero_grad(set_to_none=True)
        opt_fus.zero_grad(set_to_none=True)
    for a, b in zip(p_ref, p_fus):
        torch.testing.assert_close(b, a, rtol=2e-6, atol=1e-7)


def test_fused_adamw_step_counters_skipped_grads_and_state_dict():
    """The step counters (0-dim views of one buffer) advance only for parameters that have a
    gradient, in mixed groups the kernel and torch's step share, and survive a state-dict round
    trip into a new optimizer; values and counts stay torch's."""
    print("fused adamw counters", flush=True)
    base = _params(3)[:4]
    p_ref = [torch.nn.Parameter(t.clone()) for t in base] + [
        torch.nn.Parameter(torch.randn(9, device="cuda", dtype=torch.bfloat16))]
    p_fus = [torch.nn.Parameter(t.detach().clone()) for t in p_ref]
    opt_ref = torch.optim.AdamW(p_ref, lr=2e-3, weight_decay=0.01, foreach=False)
    opt_fus = FusedAdamW(p_fus, lr=2e-3, weight_decay=0.01)
    g = torch.Generator(device="cuda").manual_seed(4)
    for step in range(6):
        if step == 3:  # continue in a new optimizer from the saved state
            sd = opt_fus.state_dict()
            opt_fus = FusedAdamW(p_fus, lr=2e-3, weight_decay=0.01)
            opt_fus.load_state_dict(sd)
        for i, (a, b) in enumerate(zip(p_ref, p_fus)):
            skip = (i == 1 and step in (1, 4)) or (i == 4 and step == 2)
            grad = None if skip else torch.randn(a.shape, device="cuda", generator=g,
                                                 dtype=torch.float32).to(a.dtype)
            a.grad = None if grad is None else grad.clone()
            b.grad = None if grad is None else grad.clone()
        opt_ref.step()
        opt_fus.step()
        for a, b in zip(p_ref, p_fus):
            assert float(opt_fus.state[b]["step"]) == float(opt_ref.state[a]["step"])
            tol = dict(rtol=2e-6, atol=1e-7) if a.dtype == torch.float32 else {}
            torch.testing.assert_close(b, a, **tol)
    assert [float(opt_fus.state[b]["step"]) for b in p_fus] == [6.0, 4.0, 6.0, 6.0, 5.0]
