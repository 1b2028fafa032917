"""qlora_lora_wgrad_noalloc (split partials in the library's own device array, no workspace)
against qlora_lora_wgrad with a caller workspace, through the C-ABI: two calls in a row, the
second on a smaller input that reuses the array the first one left its partials in. Same
split count and summation order, so the outputs must be identical bit for bit; the first is
also checked against an fp64 product to the fp32 accumulation bound."""

import pytest
import torch

from hackathon_amd import _lib

pytestmark = pytest.mark.gpu


def _operands(M, N, slots, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    pt = torch.randn(16 * slots, M, device="cuda", generator=g).to(torch.bfloat16)
    q = torch.randn(M, N, device="cuda", generator=g).to(torch.bfloat16)
    return pt, q


def _wgrad(pt, q, slots, transposed, alpha, noalloc):
    M, N = q.shape
    nc = 16 * slots
    out = torch.full((nc, N) if transposed else (N, nc), float("nan"), device="cuda")
    stream = _lib.stream_of(q)
    if noalloc:
        _lib.call("qlora_lora_wgrad_noalloc", pt.data_ptr(), pt.stride(0), q.data_ptr(),
                  q.stride(0), M, N, slots, _lib.BF16, out.data_ptr(), int(transposed),
                  float(alpha), stream)
    else:
        ws, ws_bytes = _lib.workspace("qlora_lora_wgrad_workspace_size", M, N, slots,
                                      device=q.device)
        assert ws_bytes > 0  # both cases below split the reduction
        _lib.call("qlora_lora_wgrad", pt.data_ptr(), pt.stride(0), q.data_ptr(), q.stride(0), M,
                  N, slots, _lib.BF16, out.data_ptr(), int(transposed), float(alpha),
                  _lib.ptr(ws), ws_bytes, stream)
    return out


@pytest.mark.parametrize("order", ["large_then_small"])
def test_noalloc_wgrad_matches_the_workspace_entry_point(order):
    cases = [(4096, 3584, 3, False, 2.0), (1024, 512, 1, True, 0.5)]  # 10.5 MiB, then 0.25 MiB
    for i, (M, N, slots, transposed, alpha) in enumerate(cases):
        print(f"lora_wgrad_noalloc call {i}: M={M} N={N} slots={slots} transposed={transposed}",
              flush=True)
        pt, q = _operands(M, N, slots, seed=i)
        want = _wgrad(pt, q, slots, transposed, alpha, noalloc=False)
        got = _wgrad(pt, q, slots, transposed, alpha, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        if i == 0:
            ref = alpha * (q.double().t() @ pt.double().t())  # [N, 16 slots]
            ref = ref.t() if transposed else ref
            # worst-case fp32 summation bound: M roundings of at most 2^-24 of the sum of |terms|
            mag = abs(alpha) * (q.double().abs().t() @ pt.double().abs().t())
            mag = mag.t() if transposed else mag
            assert torch.all((got.double() - ref).abs() <= M * 2.0 ** -24 * mag + 1e-6)
