"""AdamW over the LoRA parameters in one HIP launch (`qlora_adamw_fp32`).

The reference trains the adapters with the trainer's torch AdamW: decoupled weight decay,
bias-corrected moments (torch/optim/adamw.py, `_single_tensor_adamw` / `_multi_tensor_adamw`).
`FusedAdamW` keeps that optimizer's interface and state layout (`step`, `exp_avg`,
`exp_avg_sq` per parameter, so state dicts load either way) and its per-element arithmetic,
but updates every fp32 parameter of a group with one kernel that reads p, g, m, v once and
writes p, m, v once. Parameters that are not fp32 CUDA tensors with fp32 gradients, or the
options the kernel does not implement (amsgrad, maximize, capturable, differentiable), go
through torch's own AdamW step.
"""

from __future__ import annotations

import torch

from . import _lib

_DESC_FIELDS = 6  # param, grad, exp_avg, exp_avg_sq, numel, first_chunk (ql_adamw_tensor)


class FusedAdamW(torch.optim.Optimizer):
    """torch.optim.AdamW(params, lr, betas, eps, weight_decay) on the gfx950 AdamW kernel."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2,
                 amsgrad=False, *, maximize=False):
        if lr < 0.0 or eps < 0.0 or weight_decay < 0.0:
            raise ValueError("lr, eps and weight_decay must be non-negative")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError(f"invalid betas {betas}")
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, amsgrad=amsgrad,
                        maximize=maximize)
        super().__init__(params, defaults)
        self._tables = {}
        self._counter_cache = {}

    @staticmethod
    def _fused_ok(p, group):
        g = p.grad
        return (p.is_cuda and p.dtype == torch.float32 and g is not None
                and g.dtype == torch.float32 and not g.is_sparse and p.is_contiguous()
                and g.is_contiguous() and not group["amsgrad"] and not group["maximize"])

    def _table(self, device, entries):
        """Device descriptor table for `entries` [(p, g, m, v)], rebuilt only when a pointer
        changes (gradients set to None and re-created give new ones)."""
        chunk = int(_lib.load().qlora_adamw_chunk_elems())
        key = tuple((p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), p.numel())
                    for p, g, m, v in entries)
        hit = self._tables.get(device)
        if hit is not None and hit[0] == key:
            return hit[1], hit[2]
        rows, first = [], 0
        for p, g, m, v in entries:
            rows.append([p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), p.numel(), first])
            first += (p.numel() + chunk - 1) // chunk
        host = torch.tensor(rows, dtype=torch.int64).reshape(-1, _DESC_FIELDS).pin_memory()
        table = host.to(device, non_blocking=True)
        self._tables[device] = (key, table, first)
        return table, first

    def _counters(self, group):
        """(buffer, views, slot of each parameter) for `group`: the parameters' `step` counters
        as 0-dim views of one fp32 CPU tensor, so one step advances them all with a single op
        (torch keeps one scalar tensor per parameter and adds to each: about 3.5 us apiece, a
        millisecond and more per step at 392 adapter tensors, while the GPU waits). Counters
        that are not the cached views (state loaded from a state dict, a new parameter group)
        are folded into a fresh buffer first; the views are 0-dim fp32 CPU tensors like torch's,
        so a state dict saves and loads either way."""
        params = group["params"]
        hit = self._counter_cache.get(id(group))
        if hit is not None and hit[0] is params and len(hit[2]) == len(params):
            _, buf, views, slots = hit
            stale = False
            for p in params:
                st = self.state.get(p)  # no insertion into the state's defaultdict
                if st and "step" in st and st["step"] is not views[slots[p]]:
                    stale = True
                    break
            if not stale:
                return buf, views, slots
        buf = torch.zeros(len(params), dtype=torch.float32)
        views = [buf[i] for i in range(len(params))]
        slots = {p: i for i, p in enumerate(params)}
        for p, i in slots.items():
            st = self.state.get(p)
            if st and "step" in st:
                buf[i] = float(st["step"])
                st["step"] = views[i]
        self._counter_cache[id(group)] = (params, buf, views, slots)
        return buf, views, slots

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            beta1, beta2 = group["betas"]
            lr, wd, eps = group["lr"], group["weight_decay"], group["eps"]
            buf, views, slots = self._counters(group)
            fused, other = [], []
            for p in group["params"]:
                if p.grad is None:
                    continue
                state = self.state[p]
                if len(state) == 0:
                    state["step"] = views[slots[p]]
                    state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    if group["amsgrad"]:
                        state["max_exp_avg_sq"] = torch.zeros_like(
                            p, memory_format=torch.preserve_format)
                (fused if self._fused_ok(p, group) else other).append(p)
            if fused:
                # torch's step adds one to each updated parameter's counter before using it; the
                # parameters left to torch's own step (`other`) are counted there
                if len(fused) == len(group["params"]):
                    buf += 1
                else:
                    buf[torch.tensor([slots[p] for p in fused])] += 1
                counts = buf.tolist()
                by_step = {}
                for p in fused:
                    st = self.state[p]
                    by_step.setdefault((p.device, counts[slots[p]]), []).append(
                        (p, p.grad, st["exp_avg"], st["exp_avg_sq"]))
                for (device, step), entries in by_step.items():
                    table, n_chunks = self._table(device, entries)
                    bc1 = 1.0 - beta1 ** step
                    bc2 = 1.0 - beta2 ** step
                    _lib.call("qlora_adamw_fp32", table.data_ptr(), len(entries), n_chunks,
                              1.0 - lr * wd, beta2, 1.0 - beta1, 1.0 - beta2, lr / bc1,
                              bc2 ** 0.5, eps, torch.cuda.current_stream(device).cuda_stream)
            if other:
                self._torch_step(group, other)
        return loss

    def _torch_step(self, group, params):
        """torch's AdamW for the parameters the kernel does not take (same state layout)."""
        from torch.optim.adamw import adamw

        grads, exp_avgs, exp_avg_sqs, steps = [], [], [], []
        for p in params:
            st = self.state[p]
            grads.append(p.grad)
            exp_avgs.append(st["exp_avg"])
            exp_avg_sqs.append(st["exp_avg_sq"])
            steps.append(st["step"])
        beta1, beta2 = group["betas"]
        max_sq = [self.state[p]["max_exp_avg_sq"] for p in params] if group["amsgrad"] else []
        adamw(params, grads, exp_avgs, exp_avg_sqs, max_sq, steps, amsgrad=group["amsgrad"],
              beta1=beta1, beta2=beta2, lr=group["lr"], weight_decay=group["weight_decay"],
              eps=group["eps"], maximize=group["maximize"], foreach=False)
