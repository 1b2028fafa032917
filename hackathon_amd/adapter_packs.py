"""Every adapter group of a model packed in one launch per model forward.

The fused LoRA paths multiply in the compute dtype and need, per adapter group, the packed
operands qlora_lora_pack_group writes from the fp32 factors (A, A^T|0, s*B|0, B^T: the casts
inside solution/lora.py:172's nn.Linear calls). Packed one group at a time that is 112 small
launches for a 28-layer Qwen2 step (four groups a layer), mostly launch latency.

Here a model forward is a scope (`scope`, entered by the patched Qwen2Model.forward). The
first group a scope asks for triggers the packing of every group this model asked for in
earlier forwards, in one qlora_lora_pack_jobs launch into one buffer, from the factors' values
at that moment; the later requests of the scope get their views. Packs are never reused
across forwards, so a parameter changed between two forwards by any means (an optimizer, a
state-dict load, a write through .data) is packed afresh, and a backward always reads the
packs of its own forward (each forward's buffer is its own allocation, kept by the autograd
contexts that saved its views). A group first seen in a scope, a request outside any scope
(a layer called on its own, activation-checkpointing's recompute inside the backward) and
factors that are not fp32 and contiguous are packed on their own as before; the values are
the same either way (tests/test_gpu_adapter_packs.py).
"""

from __future__ import annotations

import contextlib
import threading
import weakref

import torch

from . import _lib
from . import gemm as _gemm

_ALIGN = 256
_local = threading.local()
# model key -> _Model; an entry lives as long as its model
_REGISTRY: dict = {}


class _Group:
    """A group a model packs: weak references to its factors, their scalings, the dtype and
    padding of its packs."""

    __slots__ = ("refs", "scalings", "dtype", "pad")

    def __init__(self, factors, dtype, pad):
        self.refs = tuple((weakref.ref(a), weakref.ref(b)) for a, b, _ in factors)
        self.scalings = tuple(float(s) for _, _, s in factors)
        self.dtype = dtype
        self.pad = pad

    def factors(self):
        out = []
        for (ra, rb), s in zip(self.refs, self.scalings):
            a, b = ra(), rb()
            if a is None or b is None:
                return None
            out.append((a, b, s))
        return out


class _Plan:
    """One launch: the device job table of a set of groups (one dtype, pad and device), the
    output buffer's size and each group's output shapes and element offsets."""

    __slots__ = ("table", "njobs", "max_items", "nbytes", "slots", "dtype", "pad", "device")


class _Model:
    """What a model packs: its groups, and the plans built for their current storage."""

    __slots__ = ("groups", "signature", "plans", "slot_plan")

    def __init__(self):
        self.groups = {}      # group key -> _Group
        self.signature = None
        self.plans = []
        self.slot_plan = {}   # group key -> (plan index, shapes, element offsets)


class _Scope:
    __slots__ = ("key", "bufs")

    def __init__(self, key):
        self.key = key
        self.bufs = None  # one 16-bit buffer per plan, once packed


def _model_key(model):
    key = id(model)
    if key not in _REGISTRY:
        _REGISTRY[key] = _Model()
        weakref.finalize(model, _REGISTRY.pop, key, None)
    return key


@contextlib.contextmanager
def scope(model):
    """One forward of `model`: its adapter packs are made together at the first request."""
    prev = getattr(_local, "scope", None)
    _local.scope = _Scope(_model_key(model))
    try:
        yield
    finally:
        _local.scope = prev


def _group_key(factors, dtype, pad):
    return tuple((id(a), id(b), s) for a, b, s in factors) + (dtype, pad)


def _batchable(factors, dtype):
    a0 = factors[0][0]
    if dtype not in (torch.bfloat16, torch.float16) or not a0.is_cuda or len(factors) > 4:
        return False
    K = a0.shape[-1]
    for a, b, _ in factors:
        if (a.dtype != torch.float32 or b.dtype != torch.float32 or not a.is_contiguous()
                or not b.is_contiguous() or a.dim() != 2 or b.dim() != 2 or a.shape != (16, K)
                or b.shape[1] != 16 or a.device != a0.device or b.device != a0.device):
            return False
    return K % 8 == 0


def _signature(mdl):
    """The storage every group of `mdl` packs from (the factors' data pointers; a parameter
    given new storage, whatever its size or dtype, has a new pointer), or None when a factor
    is gone."""
    sig = []
    for grp in mdl.groups.values():
        for ra, rb in grp.refs:
            a, b = ra(), rb()
            if a is None or b is None:
                return None
            sig.append(a.data_ptr())
            sig.append(b.data_ptr())
    return tuple(sig)


def _plan(groups, dtype, pad, device):
    """A _Plan for `groups` ({group key: factors}); offsets in elements, 128-element aligned."""
    esize = torch.empty((), dtype=dtype).element_size()
    align = _ALIGN // esize
    jobs = (_lib.LoraPackJob * len(groups))()
    plan = _Plan()
    plan.slots, offset, plan.max_items = {}, 0, 0
    for j, (key, factors) in enumerate(groups.items()):
        G = len(factors)
        K = factors[0][0].shape[1]
        N = sum(b.shape[0] for _, b, _ in factors)
        shapes = ((16 * G, K), (K, pad), (N, pad), (16 * G, N))
        offs = []
        for r, c in shapes:
            offs.append(offset)
            offset += (r * c + align - 1) // align * align
        job = jobs[j]
        for g, (a, b, s) in enumerate(factors):
            job.A[g], job.B[g] = a.data_ptr(), b.data_ptr()
            job.n[g], job.scaling[g] = b.shape[0], s
        job.K, job.count = K, G
        job.a16, job.at_pad, job.bs_pad, job.bt = (o * esize for o in offs)
        plan.max_items = max(plan.max_items, (K + N) * (pad // 8) + N + 2 * G * K)
        plan.slots[key] = (shapes, offs)
    host = torch.frombuffer(bytearray(bytes(jobs)), dtype=torch.uint8).pin_memory()
    plan.table = host.to(device, non_blocking=True)
    plan.njobs, plan.nbytes = len(groups), max(offset, 1) * esize
    plan.dtype, plan.pad, plan.device = dtype, pad, device
    return plan


def _replan(mdl):
    by_kind = {}
    for key, grp in list(mdl.groups.items()):
        factors = grp.factors()
        if factors is None or not _batchable(factors, grp.dtype):
            del mdl.groups[key]
            continue
        kind = (grp.dtype, grp.pad, factors[0][0].device)
        by_kind.setdefault(kind, {})[key] = factors
    mdl.plans = [_plan(groups, *kind) for kind, groups in by_kind.items()]
    mdl.slot_plan = {key: (i, shapes, offs) for i, p in enumerate(mdl.plans)
                     for key, (shapes, offs) in p.slots.items()}
    mdl.signature = _signature(mdl)


def _launch(plan):
    buf = torch.empty(plan.nbytes // 2, dtype=plan.dtype, device=plan.device)
    _lib.call("qlora_lora_pack_jobs", plan.table.data_ptr(), plan.njobs, plan.max_items,
              buf.data_ptr(), _lib.tag(plan.dtype), plan.pad, _lib.stream_of(buf))
    return buf


def _pack_all(groups, device):
    """Pack `groups` ({group key: (factors, dtype, pad)}, one dtype and pad) in one launch:
    {group key: (a16, at_pad, bs_pad, bt)}."""
    dtype, pad = next(iter(groups.values()))[1:]
    plan = _plan({k: f for k, (f, _, _) in groups.items()}, dtype, pad, device)
    buf = _launch(plan)
    return {key: _views(buf, shapes, offs) for key, (shapes, offs) in plan.slots.items()}


def _views(buf, shapes, offs):
    return tuple(buf.as_strided((r, c), (c, 1), o) for (r, c), o in zip(shapes, offs))


def _pack_scope(sc):
    mdl = _REGISTRY.get(sc.key)
    sc.bufs = []
    if mdl is None or not mdl.groups:
        return
    if mdl.signature is None or _signature(mdl) != mdl.signature:
        _replan(mdl)
    sc.bufs = [_launch(p) for p in mdl.plans]


def pack_group(factors, dtype, pad):
    """(a16, at_pad, bs_pad, bt) of `factors` [(A [16, K], B [n_g, 16], scaling)], as
    gemm.lora_pack_group returns them: from this forward's batch when the model is inside a
    scope and asked for this group before, else packed now."""
    sc = getattr(_local, "scope", None)
    if sc is None:
        return _gemm.lora_pack_group(factors, dtype, pad)
    key = _group_key(factors, dtype, pad)
    if sc.bufs is None:
        _pack_scope(sc)
    mdl = _REGISTRY[sc.key]
    hit = mdl.slot_plan.get(key)
    if hit is not None and sc.bufs:
        i, shapes, offs = hit
        return _views(sc.bufs[i], shapes, offs)
    if key not in mdl.groups and _batchable(factors, dtype):
        mdl.groups[key] = _Group(factors, dtype, pad)   # packed with the others from the next forward
    return _gemm.lora_pack_group(factors, dtype, pad)


def pack(a, b, scaling, dtype, pad):
    """pack_group for one adapter: (a16, at_pad, bs_pad, bt), as gemm.lora_pack returns them."""
    return pack_group([(a, b, scaling)], dtype, pad)


def patch():
    """Wrap Qwen2Model.forward in a scope (idempotent)."""
    from transformers.models.qwen2 import modeling_qwen2 as m

    prev = m.Qwen2Model.forward
    if getattr(prev, "_solution_adapter_packs", False):
        return

    def forward(self, *args, **kwargs):
        with scope(self):
            return prev(self, *args, **kwargs)

    forward._solution_patch = True
    forward._solution_adapter_packs = True
    forward._original = prev
    forward.__wrapped__ = prev
    m.Qwen2Model.forward = forward
