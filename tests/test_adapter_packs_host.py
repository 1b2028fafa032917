"""Host logic of adapter_packs (no GPU): the forward scope, the per-model registry and the
fallback to one pack per group."""

import gc

import torch

from hackathon_amd import adapter_packs
from hackathon_amd import gemm as _gemm


class _Model(torch.nn.Module):
    pass


def test_scopes_nest_and_restore():
    outer, inner = _Model(), _Model()
    assert getattr(adapter_packs._local, "scope", None) is None
    with adapter_packs.scope(outer):
        s1 = adapter_packs._local.scope
        assert s1.key == id(outer) and s1.bufs is None
        with adapter_packs.scope(inner):
            assert adapter_packs._local.scope.key == id(inner)
        assert adapter_packs._local.scope is s1
    assert adapter_packs._local.scope is None


def test_registry_entry_lives_as_long_as_its_model():
    m = _Model()
    with adapter_packs.scope(m):
        pass
    key = id(m)
    assert key in adapter_packs._REGISTRY
    del m
    gc.collect()
    assert key not in adapter_packs._REGISTRY


def test_outside_a_scope_each_group_is_packed_on_its_own(monkeypatch):
    calls = []
    monkeypatch.setattr(_gemm, "lora_pack_group",
                        lambda factors, dtype, pad: calls.append((len(factors), dtype, pad)) or "packed")
    a, b = torch.zeros(16, 64), torch.zeros(32, 16)
    assert adapter_packs.pack(a, b, 2.0, torch.bfloat16, 64) == "packed"
    assert calls == [(1, torch.bfloat16, 64)]


def test_cpu_or_non_fp32_factors_are_not_batched(monkeypatch):
    monkeypatch.setattr(_gemm, "lora_pack_group", lambda factors, dtype, pad: "packed")
    a, b = torch.zeros(16, 64), torch.zeros(32, 16)
    assert not adapter_packs._batchable([(a, b, 2.0)], torch.bfloat16)
    m = _Model()
    with adapter_packs.scope(m):
        assert adapter_packs.pack(a, b, 2.0, torch.bfloat16, 64) == "packed"
        # a factor set the batch cannot take is never registered
        assert not adapter_packs._REGISTRY[id(m)].groups
