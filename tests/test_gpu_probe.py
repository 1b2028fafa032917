"""qlora_mfma_probe, the measurement-only entry point behind bench.py --workload gemm_data: every
mode runs, zero operands give zero accumulators where the products only see them (modes 0 and
1: with the loads of modes 2 and 3 the second stage holds the source's data), N(0,1) operands
give finite sums, and bad arguments are refused."""

import pytest
import torch

from hackathon_amd import _lib

pytestmark = pytest.mark.gpu


def _probe(ops, mode, iters, wgs, out, src):
    _lib.call("qlora_mfma_probe", ops.data_ptr(), _lib.tag(torch.bfloat16), mode, iters, wgs,
              out.data_ptr(), src.data_ptr(), _lib.stream_of(out))


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_mfma_probe_modes(mode):
    print(f"mfma probe mode {mode}", flush=True)
    wgs = 8
    out = torch.full((256 * wgs,), float("nan"), device="cuda")
    src = torch.randn(2 << 19, device="cuda").to(torch.bfloat16)
    zeros = torch.zeros(1024 * 8, dtype=torch.bfloat16, device="cuda")
    _probe(zeros, mode, 6, wgs, out, src)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    if mode < 2:
        assert torch.equal(out, torch.zeros_like(out))
    g = torch.Generator(device="cuda").manual_seed(0)
    ops = torch.randn(1024 * 8, device="cuda", generator=g).to(torch.bfloat16)
    _probe(ops, mode, 6, wgs, out, src)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and out.abs().sum() > 0


def test_mfma_probe_rejects_bad_arguments():
    out = torch.empty(256, device="cuda")
    ops = torch.zeros(1024 * 8, dtype=torch.bfloat16, device="cuda")
    for mode, iters, wgs in ((4, 1, 1), (0, 0, 1), (0, 1, 0), (0, 1, 70000)):
        with pytest.raises(RuntimeError):
            _probe(ops, mode, iters, wgs, out, ops)
    with pytest.raises(RuntimeError):  # modes 2 and 3 need a source
        _lib.call("qlora_mfma_probe", ops.data_ptr(), _lib.tag(torch.bfloat16), 2, 1, 1,
                  out.data_ptr(), None, _lib.stream_of(out))
