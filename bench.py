#!/usr/bin/env python3
"""Benchmark of the gfx950 QLoRA kernel set on one MI355X; prints ONE JSON line.

Headline (`value`): NF4 dequant HBM GB/s on the Qwen2.5-7B gate/up projection weight
(18944 x 3584, NF4 blocksize 64, absmax double-quantised with blocksize 256, bf16 output),
the dequant the 7B QLoRA step runs 392 times per step. A step = one dequant of one weight;
`--sets` weight/output buffer sets (4 x 171 MB by default) are rotated so the working set
exceeds the 256 MB Infinity Cache and every step streams from HBM. Inputs are resident in
HBM before the timed region; the K steps are captured in one HIP graph and replayed, timed
with HIP events on the stream the kernels run on.

Also reported in the same line:
  roofline       the dequant kernel against the 8 TB/s HBM peak (algorithmic bytes/launch);
                 `traffic` is the stored rocprofv3 FETCH+WRITE figure (not measured here)
  cpu_baseline   the reference path's dequant on the host CPU: the oracle's torch restatement
                 on every host thread, Qwen2.5-0.5B gate_proj weight, bounded sample; the C
                 oracle on one thread is reported beside it (cpu_baseline_c_1thread)
  cpu_baselines  the other workloads' CPU side on the host (oracle torch restatements and the
                 eager model path), bounded samples with stated extrapolation
  nf4_4864x896   the same dequant on the Qwen2.5-0.5B gate_proj weight (32 rotated sets), with
                 the graph launch floor (an empty kernel's per-launch time) and a plain copy
                 and fill of the same 10.97 MB, timed the same way, beside it
  kernels        per-kernel device time and roofline of the other kernels at their shapes,
                 and the Qwen2.5-7B LoRA MLP forward + backward at 4096 tokens (patched vs
                 eager, TFLOP/s against 3.364 TFLOP of work)
  qlora_step     Qwen2.5-7B-shaped QLoRA training step tokens/s, patched vs PyTorch eager
  qlora_step_dropout  the same step with LoRA dropout 0.05 on every adapter

`python bench.py --gpus N --steps K --warmup W`; N > 1 is not run (one GPU only).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
METRIC = "NF4 dequant HBM GB/s (% peak); QLoRA step tokens/s at Qwen2.5-7B shape"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def nf4_algorithmic_bytes(n, blocksize=64, blocksize2=256):
    """Bytes one dequant call must move: packed nibbles n/2, absmax codes n/bs, second-level
    scales 4*ceil(nblocks/bs2), bf16 output 2n, plus the 256-entry code2 and 16-entry NF4
    tables (1088 B)."""
    nb = math.ceil(n / blocksize)
    return n // 2 + nb + 4 * math.ceil(nb / blocksize2) + 2 * n + 1088


# ---------------------------------------------------------------------------------------------
def _graph_time(fn_list, torch, replays=1):
    """Capture the calls in one HIP graph, replay once to warm, then time `replays` replays with
    events on the current stream. Returns seconds per call."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for f in fn_list[:2]:
            f()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fn_list:
            f()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / (replays * len(fn_list))


def bench_nf4(torch, shape, steps, warmup, sets, seed=0):
    from hackathon_amd import nf4, quant

    n = shape[0] * shape[1]
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(shape, device="cuda", generator=g) * 0.02
    packed, st = quant.quantize_nf4(w, 64, compress_statistics=True)
    del w
    bufs = []
    for i in range(sets):
        p = packed.clone()
        s = quant.QuantState(st.absmax.clone(), st.shape, st.code, st.blocksize, offset=st.offset,
                             state2=quant.QuantState(st.state2.absmax.clone(), code=st.state2.code,
                                                     blocksize=st.state2.blocksize))
        out = torch.empty(shape, dtype=torch.bfloat16, device="cuda")
        bufs.append((p, s, out))
    for i in range(max(warmup, sets)):  # every set once: its scalars are read before capture
        p, s, o = bufs[i % sets]
        nf4.dequantize_nf4(p, s, torch.bfloat16, out=o)
    torch.cuda.synchronize()
    calls = [(lambda b=bufs[i % sets]: nf4.dequantize_nf4(b[0], b[1], torch.bfloat16, out=b[2]))
             for i in range(steps)]
    sec = _graph_time(calls, torch)
    nbytes = nf4_algorithmic_bytes(n)
    return dict(sec_per_call=sec, bytes_per_call=nbytes, gbs=nbytes / sec / 1e9, n=n)


def launch_floor(torch, steps=200, sets=32):
    """Seconds per launch of the smallest kernel (a one-element fill) captured `steps` times in
    one HIP graph and timed like the dequant: the per-launch cost any kernel pays in this
    timing, before it moves a byte. On MI355X it is about 1.6 us, with one workgroup or
    a thousand."""
    bufs = [torch.empty(1, device="cuda") for _ in range(sets)]
    return _graph_time([(lambda b=bufs[i % sets]: b.zero_()) for i in range(steps)], torch,
                       replays=3)


def same_bytes_moves(torch, nbytes, steps=200, sets=32):
    """Seconds per call of two plain kernels that move `nbytes` and nothing else, timed like
    the dequant (`steps` calls over `sets` rotated buffers in one HIP graph): a device copy
    (nbytes / 2 read, nbytes / 2 written) and a fill (nbytes written; the dequant's traffic is
    80% writes)."""
    n = nbytes // 4
    pairs = [(torch.ones(n, dtype=torch.bfloat16, device="cuda"),
              torch.empty(n, dtype=torch.bfloat16, device="cuda")) for _ in range(sets)]
    copy = _graph_time([(lambda b=pairs[i % sets]: b[1].copy_(b[0])) for i in range(steps)],
                       torch, replays=3)
    del pairs
    fills = [torch.empty(2 * n, dtype=torch.bfloat16, device="cuda") for _ in range(sets)]
    fill = _graph_time([(lambda b=fills[i % sets]: b.fill_(1.0)) for i in range(steps)], torch,
                       replays=3)
    return copy, fill


def bench_nf4_small(torch, steps=200, warmup=5):
    """The dequant on the Qwen2.5-0.5B gate_proj weight (4864 x 896, 10.97 MB per call, 32
    rotated sets) beside the launch floor and beside plain kernels moving the same bytes in
    the same timing: `above_floor_gbs` is the rate of the time the dequant adds to an empty
    launch; `copy_same_bytes_us` / `fill_same_bytes_us` are a device copy and a fill of the
    same 10.97 MB. 70% of HBM peak would be 1.96 us per call."""
    r = bench_nf4(torch, (4864, 896), steps, warmup, 32, seed=1)
    floor = launch_floor(torch, steps)
    copy, fill = same_bytes_moves(torch, r["bytes_per_call"], steps)
    extra = r["sec_per_call"] - floor
    nb = r["bytes_per_call"]
    return dict(us=round(r["sec_per_call"] * 1e6, 3), gbs=round(r["gbs"], 1),
                frac_hbm=round(r["gbs"] / HBM_PEAK_GBS, 4), bytes=nb,
                rotated_sets=32, launch_floor_us=round(floor * 1e6, 3),
                above_floor_gbs=round(nb / extra / 1e9, 1) if extra > 0 else None,
                copy_same_bytes_us=round(copy * 1e6, 3),
                copy_same_bytes_frac_hbm=round(nb / copy / 1e9 / HBM_PEAK_GBS, 4),
                fill_same_bytes_us=round(fill * 1e6, 3),
                fill_same_bytes_frac_hbm=round(nb / fill / 1e9 / HBM_PEAK_GBS, 4))


def cpu_baseline_nf4(seconds, shape=(4864, 896), threads=None):
    """The reference path's dequant on the host: the oracle's vectorised torch restatement
    (oracle/nf4.py dequant_torch, bit-exact to the C oracle) on `threads` intra-op threads
    (default: every host CPU), dequantising the Qwen2.5-0.5B gate_proj weight repeatedly for
    about `seconds`. Returns GB/s of algorithmic bytes."""
    import numpy as np
    import torch

    from hackathon_amd import quant
    from oracle import nf4 as onf4

    threads = threads or os.cpu_count()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        g = torch.Generator().manual_seed(0)
        w = torch.randn(shape, generator=g) * 0.02
        packed, st = quant.quantize_nf4(w, 64, compress_statistics=True)
        table = np.array(quant.NF4_CODE, dtype=np.float32)
        n = shape[0] * shape[1]
        onf4.dequant_torch(packed, st, table)
        reps, t0 = 0, time.perf_counter()
        while True:
            onf4.dequant_torch(packed, st, table)
            reps += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
    finally:
        torch.set_num_threads(prev)
    nbytes = nf4_algorithmic_bytes(n)
    return dict(value=round(nbytes * reps / el / 1e9, 3), unit="GB/s", cores=threads,
                kind="port",
                sample=f"torch CPU restatement of the reference dequant (oracle dequant_torch, "
                       f"bit-exact to the C oracle) of a {shape[0]}x{shape[1]} weight to bf16, "
                       f"{reps} repetitions in {el:.1f} s on {threads} threads")


def cpu_baseline_nf4_c(seconds, shape=(4864, 896)):
    """The C oracle (one host thread) on the same weight, for comparison."""
    import numpy as np
    import torch

    from hackathon_amd import quant
    from oracle import nf4 as onf4

    g = torch.Generator().manual_seed(0)
    w = torch.randn(shape, generator=g) * 0.02
    packed, st = quant.quantize_nf4(w, 64, compress_statistics=True)
    table = np.array(quant.NF4_CODE, dtype=np.float32)
    n = shape[0] * shape[1]
    reps, t0 = 0, time.perf_counter()
    while True:
        onf4.dequant_state(packed, st, table, out="bf16")
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    nbytes = nf4_algorithmic_bytes(n)
    return dict(value=round(nbytes * reps / el / 1e9, 3), unit="GB/s", cores=1, kind="port",
                sample=f"C oracle nf4 dequant of a {shape[0]}x{shape[1]} weight (bf16 out), "
                       f"{reps} repetitions in {el:.1f} s on one host thread")


def cpu_baselines(torch):
    """The reference path's CPU side at the other configs, timed on the host beside the GPU
    run (reported baselines, not targets): the oracle's torch restatements of RMSNorm, RoPE
    and the unfused lm_head + cross-entropy (oracle/ops.py), and the plain PyTorch path of a
    Qwen2.5-7B-shaped layer (the eager model path, torch-op NF4 dequant, LoRA, attention) for
    the MLP and the step. Each runs a bounded sample, and the extrapolation is stated."""
    import torch.nn.functional as F

    from hackathon_amd import qlora_step
    from oracle import ops

    def tm(fn, min_s=0.5):
        fn()
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= min_s:
                return el / n

    g = torch.Generator().manual_seed(0)
    bf = torch.bfloat16
    res = {"cores": torch.get_num_threads(), "kind": "port", "host_cpu": _cpu_model()}
    # RMSNorm 4 x 2048 x 1536 and RoPE q 4x12x2048x128 / k 4x2x2048x128, full shape
    x = torch.randn(8192, 1536, generator=g).to(bf)
    w = (1 + 0.1 * torch.randn(1536, generator=g)).to(bf)
    dy = torch.randn(8192, 1536, generator=g).to(bf)
    _, rstd = ops.rmsnorm_fwd(x, w, 1e-6)
    for name, fn, nbytes in (("rmsnorm_fwd_8192x1536", lambda: ops.rmsnorm_fwd(x, w, 1e-6),
                              50_367_488),
                             ("rmsnorm_bwd_8192x1536", lambda: ops.rmsnorm_bwd(dy, x, w, rstd),
                              75_533_312)):
        t = tm(fn)
        res[name] = dict(ms=round(t * 1e3, 2), gbs=round(nbytes / t / 1e9, 2), sample="full shape")
    q = torch.randn(4, 2048, 12, 128, generator=g).to(bf).transpose(1, 2)
    k = torch.randn(4, 2048, 2, 128, generator=g).to(bf).transpose(1, 2)
    cos, sin = ops.qwen_cos_sin(1, 2048, 128, dtype=bf)
    t = tm(lambda: ops.rope(q, k, cos, sin))
    res["rope_fwd_4x2048x(12+2)x128"] = dict(ms=round(t * 1e3, 2),
                                             gbs=round(59_768_832 / t / 1e9, 2),
                                             sample="full shape")
    del x, w, dy, q, k
    # full-logits lm_head + cross-entropy forward and dz @ W on 256 of the 8192 rows
    rows, H, V = 256, 1536, 151936
    W32 = (torch.randn(V, H, generator=g) * 0.02).to(bf).float()
    h = torch.randn(rows, H, generator=g).to(bf).float().requires_grad_()
    tgt = torch.randint(0, V, (rows,), generator=g)
    tgt[torch.rand(rows, generator=g) < 0.1] = -100

    def ce():
        h.grad = None
        F.cross_entropy(h @ W32.t(), tgt, ignore_index=-100).backward()
    t = tm(ce, 1.0) * (8192 / rows)
    fl = 2 * 2.0 * 8192 * H * V
    res["fused_ce_8192x1536x151936"] = dict(
        ms=round(t * 1e3, 1), tflops=round(fl / t / 1e12, 3),
        sample=f"{rows} of 8192 rows (fp32 full logits), scaled linearly by rows")
    ce_rate = fl / t
    del W32, h
    # the 7B MLP and the QLoRA step: the eager PyTorch path of one Qwen2.5-7B-shaped layer on
    # the host
    cfg = qlora_step.qwen2_config(num_hidden_layers=1, vocab_size=1024)
    model = qlora_step.build_qlora_model(cfg, "cpu")
    mlp = model.model.layers[0].mlp
    gm = torch.Generator().manual_seed(1)

    def mlp_step(T):
        xm = torch.randn(1, T, cfg.hidden_size, generator=gm).to(bf).requires_grad_()
        mlp(xm).float().sum().backward()

    def model_step(T):
        ids = torch.randint(0, cfg.vocab_size, (1, T), generator=gm)
        model(input_ids=ids, labels=ids, use_cache=False).loss.backward()

    with qlora_step.eager_mode(model):
        pts = [(T, tm(lambda T=T: mlp_step(T), 1.0)) for T in (256, 1024)]
        slope = (pts[1][1] - pts[0][1]) / (pts[1][0] - pts[0][0])
        t_mlp = pts[0][1] + slope * (4096 - pts[0][0])
        res["qwen25_7b_mlp_lora_4096tok"] = dict(
            ms=round(t_mlp * 1e3, 1), tflops=round(3.3638e12 / t_mlp / 1e12, 3),
            sample="MLP fwd+bwd at 256 and 1024 tokens (NF4 dequant, LoRA, SwiGLU), "
                   "fitted a + b*tokens and evaluated at 4096")
        pts = [(T, tm(lambda T=T: model_step(T), 1.0)) for T in (512, 1024)]
        slope = (pts[1][1] - pts[0][1]) / (pts[1][0] - pts[0][0])
        t_layer = pts[0][1] + slope * (4096 - pts[0][0])
    qlora_step.patched_mode()
    head = 2 * 2.0 * 4096 * cfg.hidden_size * 152064 / ce_rate
    t_step = 28 * t_layer + head
    res["qlora_step_qwen25_7b"] = dict(
        ms=round(t_step * 1e3, 0), tokens_per_s=round(4096 / t_step, 1),
        sample="extrapolated: one decoder layer fwd+bwd (with its embedding, norm and a 1024-word "
               "head) at 512 and 1024 tokens, fitted linearly to 4096 tokens x 28 layers, plus the "
               "152064-word head at the lm_head + CE CPU rate above; attention's quadratic term is only "
               "partly in the fit, so this is a lower bound on the CPU time")
    del model, mlp
    return res


# ---------------------------------------------------------------------------------------------
MALL_BYTES = 256 * 2**20   # MI355X Infinity Cache: rotated working sets must exceed it


def _rotated_sets(bytes_per_set, minimum=5):
    """Buffer sets to rotate so that the sets together exceed the MALL (at least `minimum`)."""
    return max(minimum, math.ceil(1.25 * MALL_BYTES / bytes_per_set))


def _rate(name, t, nbytes, res):
    if nbytes / t / 1e9 > 1.25 * HBM_PEAK_GBS:  # every set exceeds the MALL: HBM bounds the rate
        raise RuntimeError(f"{name}: {nbytes / t / 1e9:.0f} GB/s is above the HBM peak; the timed "
                           f"region did not run the kernels")
    res[name] = dict(us=round(t * 1e6, 2), gbs=round(nbytes / t / 1e9, 1),
                     frac_hbm=round(nbytes / t / 1e9 / HBM_PEAK_GBS, 3), bytes=nbytes)


def bench_rmsnorm(torch, res, replays=4):
    """RMSNorm forward and backward at 4 x 2048 x 1536 bf16 (eps 1e-6), rotating buffer sets
    larger than the MALL so every launch streams from HBM."""
    from hackathon_amd import _lib

    M, N = 8192, 1536
    g = torch.Generator(device="cuda").manual_seed(0)
    w = (1 + 0.1 * torch.randn(N, device="cuda", generator=g)).to(torch.bfloat16)
    fwd_bytes = 2 * M * N * 2 + N * 2 + M * 4
    bwd_bytes = 3 * M * N * 2 + N * 2 + M * 4
    sets = _rotated_sets(bwd_bytes)
    bufs = []
    for _ in range(sets):
        x = torch.randn(M, N, device="cuda", generator=g).to(torch.bfloat16)
        dy = torch.randn(M, N, device="cuda", generator=g).to(torch.bfloat16)
        bufs.append((x, dy, torch.empty_like(x), torch.empty(M, device="cuda"),
                     torch.empty_like(x)))
    def fwd(b):  # the stream is looked up at launch: inside graph capture it is the capture's
        x, _, y, rstd, _ = b
        _lib.call("qlora_rmsnorm_fwd", x.data_ptr(), 2, N, w.data_ptr(), 2, y.data_ptr(), 2, N,
                  rstd.data_ptr(), M, N, 1e-6, _lib.stream_of(x))

    def bwd(b):
        x, dy, _, rstd, dx = b
        _lib.call("qlora_rmsnorm_bwd", dy.data_ptr(), 2, N, x.data_ptr(), 2, N, w.data_ptr(), 2,
                  rstd.data_ptr(), dx.data_ptr(), 2, N, M, N, _lib.stream_of(x))
    for b in bufs:
        fwd(b)
    calls = 4 * sets
    t = _graph_time([lambda b=bufs[i % sets]: fwd(b) for i in range(calls)], torch, replays)
    _rate("rmsnorm_fwd_8192x1536", t, fwd_bytes, res)
    t = _graph_time([lambda b=bufs[i % sets]: bwd(b) for i in range(calls)], torch, replays)
    _rate("rmsnorm_bwd_8192x1536", t, bwd_bytes, res)
    res["rmsnorm_fwd_8192x1536"]["rotated_sets"] = res["rmsnorm_bwd_8192x1536"]["rotated_sets"] = sets


def bench_rope(torch, res, replays=4):
    """RoPE forward and backward of q (4,12,2048,128) and k (4,2,2048,128), (B,H,S,D) views of
    (B,S,H,D) buffers, cos/sin (1,2048,128) broadcast over the batch, theta 1e6, bf16; rotated
    buffer sets larger than the MALL."""
    from hackathon_amd import rope

    dev = "cuda"
    B, S, HQ, HK, D = 4, 2048, 12, 2, 128
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, device=dev).float() / D))
    emb = torch.cat([torch.outer(torch.arange(S, device=dev).float(), inv)] * 2, -1)
    cos, sin = emb.cos()[None].to(torch.bfloat16), emb.sin()[None].to(torch.bfloat16)
    cos_e, sin_e = cos.expand(B, S, D), sin.expand(B, S, D)
    nbytes = 2 * 2 * B * S * (HQ + HK) * D + 2 * 2 * S * D
    sets = _rotated_sets(nbytes)
    g = torch.Generator(device=dev).manual_seed(0)
    bufs = []
    for _ in range(sets):
        q = torch.randn(B, S, HQ, D, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
        k = torch.randn(B, S, HK, D, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
        bufs.append((q, k, torch.empty_like(q), torch.empty_like(k)))
    calls = 4 * sets
    for name, backward in (("rope_fwd_4x2048x(12+2)x128", False),
                           ("rope_bwd_4x2048x(12+2)x128", True)):
        fns = [lambda b=bufs[i % sets], bw=backward: rope._launch(b[0], b[1], cos_e, sin_e, b[2],
                                                                  b[3], bw)
               for i in range(calls)]
        t = _graph_time(fns, torch, replays)
        _rate(name, t, nbytes, res)
        res[name]["rotated_sets"] = sets


def bench_swiglu(torch, res):
    """SwiGLU forward and backward at the 7B MLP, 4096 x 18944 bf16 (465.6 / 775.9 MB per
    call, more than the MALL)."""
    from hackathon_amd import _lib

    n = 4096 * 18944
    g = torch.Generator(device="cuda").manual_seed(0)
    gt = torch.randn(n, device="cuda", generator=g).to(torch.bfloat16)
    up = torch.randn(n, device="cuda", generator=g).to(torch.bfloat16)
    o = torch.empty_like(gt)
    gr = torch.randn(n, device="cuda", generator=g).to(torch.bfloat16)
    dg, du = torch.empty_like(gt), torch.empty_like(gt)

    def s():  # looked up at launch: inside graph capture it is the capture's stream
        return _lib.stream_of(gt)
    for name, fn, nbytes in (
            ("swiglu_fwd_4096x18944", lambda: _lib.call("qlora_swiglu_fwd", gt.data_ptr(),
                                                       up.data_ptr(), o.data_ptr(), 2, n, s()),
             3 * 2 * n),
            ("swiglu_bwd_4096x18944", lambda: _lib.call("qlora_swiglu_bwd", gr.data_ptr(),
                                                       gt.data_ptr(), up.data_ptr(), dg.data_ptr(),
                                                       du.data_ptr(), 2, n, s()), 5 * 2 * n)):
        _rate(name, _graph_time([fn] * 10, torch, replays=3), nbytes, res)
    # the backward fused with the gate and up adapters' down-projections (the LoRA MLP's
    # backward): the same 775.9 MB plus B^T of both adapters (1.2 MB) and du, du^T (0.8 MB)
    from hackathon_amd import gemm, swiglu

    M, N = 4096, 18944
    bt = (torch.randn(32, N, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    dlo = torch.empty(M, 64, device="cuda", dtype=torch.bfloat16)
    dlo_t = gemm.lora_t_buffer(M, torch.bfloat16, "cuda", rows=32)
    views = [t.view(M, N) for t in (gr, gt, up, dg, du)]

    def fused():
        swiglu.swiglu_bwd_lora_down(*views, bt[:16], bt[16:], 1.0, 1.0, dlo, dlo_t)
    _rate("swiglu_bwd_lora_down_4096x18944", _graph_time([fused] * 10, torch, replays=3),
          5 * 2 * n + 2 * 32 * N + 2 * (M * 64 + 32 * M), res)
    # ... and with both adapters' lora_B gradients in the same pass: plus u^T of both adapters
    # (0.3 MB) and the two fp32 [18944, 16] gradients (2.4 MB)
    ut = gemm.lora_t_buffer(M, torch.bfloat16, "cuda", rows=32)
    ut.copy_(torch.randn(32, M, device="cuda", generator=g).to(torch.bfloat16))

    def fused_db():
        swiglu.swiglu_bwd_lora(*views, bt[:16], bt[16:], ut[:16], ut[16:32], 1.0, 1.0, 1.0, 1.0,
                               dlo, dlo_t)
    _rate("swiglu_bwd_lora_4096x18944", _graph_time([fused_db] * 10, torch, replays=3),
          5 * 2 * n + 2 * 32 * N + 2 * 32 * M + 2 * (M * 64 + 32 * M) + 2 * 4 * 16 * N, res)
    # ... and with the down adapter's lora_A gradient du_d^T h too (h recomputed on chip): plus
    # du_d^T (0.1 MB) and the fp32 [16, 18944] gradient (1.2 MB)
    udt = gemm.lora_t_buffer(M, torch.bfloat16, "cuda", rows=16)
    udt.copy_(torch.randn(16, M, device="cuda", generator=g).to(torch.bfloat16))

    def fused_da():
        swiglu.swiglu_bwd_lora(*views, bt[:16], bt[16:], ut[:16], ut[16:32], 1.0, 1.0, 1.0, 1.0,
                               dlo, dlo_t, ud_t=udt)
    _rate("swiglu_bwd_lora_da_4096x18944", _graph_time([fused_da] * 10, torch, replays=3),
          5 * 2 * n + 2 * 32 * N + 2 * 48 * M + 2 * (M * 64 + 32 * M) + 3 * 4 * 16 * N, res)
    # the forward fused with the down adapter's u = h A^T: the SwiGLU forward's 465.6 MB plus A
    # (0.6 MB) and u, u^T (0.7 MB)
    a16 = (torch.randn(16, N, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    u16 = torch.empty(M, 64, device="cuda", dtype=torch.bfloat16)
    u16_t = gemm.lora_t_buffer(M, torch.bfloat16, "cuda", rows=16)
    hv = dg.view(M, N)

    def fused_fwd():
        swiglu.swiglu_fwd_lora_down(views[1], views[2], hv, a16, u16, u16_t)
    _rate("swiglu_fwd_lora_down_4096x18944", _graph_time([fused_fwd] * 10, torch, replays=3),
          3 * 2 * n + 2 * 16 * N + 2 * (M * 64 + 16 * M), res)


def bench_gemms(torch, res):
    """The MLP's GEMM shapes: x[4096,3584] @ W[18944,3584]^T and dY[4096,18944] @ W, beside
    hipBLASLt through torch.matmul on the same operands."""
    from hackathon_amd import gemm

    dev = "cuda"
    for name, (Mm, Nn, Kk, b_kn) in (("gemm_nt_4096x18944x3584", (4096, 18944, 3584, False)),
                                     ("gemm_nt_4096x3584x18944", (4096, 3584, 18944, False)),
                                     ("gemm_nn_4096x3584x18944", (4096, 3584, 18944, True))):
        a = torch.randn(Mm, Kk, device=dev).to(torch.bfloat16)
        bm = torch.randn((Kk, Nn) if b_kn else (Nn, Kk), device=dev).to(torch.bfloat16)
        c = torch.empty(Mm, Nn, device=dev, dtype=torch.bfloat16)
        t = _graph_time([lambda: gemm.gemm(a, bm, b_kn=b_kn, out=c)] * 5, torch)
        fl = 2.0 * Mm * Nn * Kk
        res[name] = dict(us=round(t * 1e6, 1), tflops=round(fl / t / 1e12, 1),
                         frac_mfma=round(fl / t / 1e12 / BF16_PEAK_TFLOPS, 3))
        ref = torch.empty_like(c)
        tt = _graph_time([lambda: torch.matmul(a, bm if b_kn else bm.t(), out=ref)] * 5, torch)
        res[name]["torch_hipblaslt_tflops"] = round(fl / tt / 1e12, 1)
        del a, bm, c, ref


def bench_ce(torch, res, reps=3):
    """Fused lm_head + cross-entropy at 8192 x 1536 x 151936 bf16 (hidden ~N(0,1), W
    ~N(0,0.02), 10% of the labels ignored): forward with the hidden gradient, 2 x 3.824 TFLOP."""
    from hackathon_amd import cross_entropy

    dev = "cuda"
    n_rows, H, V = 8192, 1536, 151936
    g = torch.Generator(device=dev).manual_seed(0)
    hid = torch.randn(n_rows, H, device=dev, generator=g).to(torch.bfloat16).requires_grad_()
    W = (torch.randn(V, H, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    tgt = torch.randint(0, V, (n_rows,), device=dev, generator=g)
    tgt[torch.rand(n_rows, device=dev, generator=g) < 0.1] = -100
    denom = (tgt != -100).sum()

    def ce_step():
        # the default chunk (512 rows, grouped by the engine up to its logits budget), as the
        # patched model's loss runs it
        loss, *_ = cross_entropy.FusedLinearCrossEntropy.apply(hid, W, tgt, denom,
                                                               torch.bfloat16,
                                                               cross_entropy.CHUNK_ROWS)
        return loss
    ce_step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        ce_step()
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / reps
    fl = 2 * 2.0 * n_rows * H * V
    res["fused_ce_8192x1536x151936"] = dict(ms=round(t * 1e3, 2), tflops=round(fl / t / 1e12, 1),
                                           frac_mfma=round(fl / t / 1e12 / BF16_PEAK_TFLOPS, 3))


def _event_time(fn, torch, calls=20, warm=3):
    """Seconds per call of `fn`, timed with events around `calls` back-to-back calls (for calls
    that allocate their outputs, which a captured graph would keep fixed)."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(calls):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / calls


def _flops(name, t, flop, res):
    res[name] = dict(us=round(t * 1e6, 2), tflops=round(flop / t / 1e12, 1),
                     frac_mfma=round(flop / t / 1e12 / BF16_PEAK_TFLOPS, 3))


def bench_next_rows(torch, res):
    """The kernels beside the six, at the shapes the Qwen2.5-7B step runs them:
    - causal flash attention, 2 x 2048 tokens, 28 query / 4 kv heads, head_dim 128, bf16:
      forward 4 B HQ S^2 D / 2 FLOP, backward 2.5x that (the algorithmic count; the kernels
      recompute P in both backward passes); inputs resident (29 MB of q);
    - the residual-add RMSNorm forward and the backward with the residual gradient, 4096 x
      3584 bf16, rotated sets;
    - the grouped NF4 dequant of the q|k|v weights (3584 + 512 + 512 rows x 3584), plain and
      transposed, rotated sets;
    - the GPU NF4 quantiser (18944 x 3584 bf16 -> NF4 bs64 with double-quant absmax);
    - the fused AdamW over the 7B adapter set (392 fp32 tensors, 40.4 M values: p, g, m, v
      read and p, m, v written, 28 B a value)."""
    import math as _m

    from hackathon_amd import _lib, attention, nf4, quant, qlora_step

    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(0)
    B, S, HQ, HK, D = 2, 2048, 28, 4, 128
    q = torch.randn(B, S, HQ, D, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
    k = torch.randn(B, S, HK, D, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
    v = torch.randn(B, S, HK, D, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
    do = torch.randn(B, S, HQ, D, device=dev, generator=g).to(torch.bfloat16)
    scale = 1.0 / _m.sqrt(D)
    o, lse = attention.attn_fwd(q, k, v, scale)
    fl = 4 * B * HQ * S * S * D / 2
    _flops("attn_fwd_2x2048x28q4kvx128", _event_time(lambda: attention.attn_fwd(q, k, v, scale),
                                                     torch), fl, res)
    _flops("attn_bwd_2x2048x28q4kvx128",
           _event_time(lambda: attention.attn_bwd(q, k, v, o, lse, do, scale), torch), 2.5 * fl,
           res)
    # torch's SDPA on the same inputs, called as transformers' eager path calls it (kv heads
    # repeated, is_causal): the forward alone, and forward + backward through autograd
    rep = HQ // HK
    kr = k.repeat_interleave(rep, dim=1).contiguous().requires_grad_()
    vr = v.repeat_interleave(rep, dim=1).contiguous().requires_grad_()
    qr = q.contiguous().requires_grad_()
    do_t = do.transpose(1, 2).contiguous()
    from torch.nn.attention import SDPBackend, sdpa_kernel

    # the fused backends only: the math fallback would run batched bf16 products on
    # transposed views
    fused_backends = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]

    def sdpa(*a, **kw):
        with sdpa_kernel(fused_backends):
            return torch.nn.functional.scaled_dot_product_attention(*a, **kw)

    def sdpa_fwd():
        with torch.no_grad():
            sdpa(qr, kr, vr, is_causal=True, scale=scale)

    def sdpa_fwd_bwd():
        out = sdpa(qr, kr, vr, is_causal=True, scale=scale)
        torch.autograd.grad(out, (qr, kr, vr), do_t)

    t_f = _event_time(sdpa_fwd, torch)
    t_fb = _event_time(sdpa_fwd_bwd, torch)
    res["torch_sdpa_2x2048x28q4kvx128"] = dict(
        fwd_us=round(t_f * 1e6, 1), fwd_tflops=round(fl / t_f / 1e12, 1),
        bwd_us=round((t_fb - t_f) * 1e6, 1), bwd_tflops=round(2.5 * fl / (t_fb - t_f) / 1e12, 1),
        note="forward + backward minus forward; kv heads repeated as transformers does")
    del q, k, v, do, o, lse, qr, kr, vr, do_t

    M, N = 4096, 3584
    w = (1 + 0.1 * torch.randn(N, device=dev, generator=g)).to(torch.bfloat16)
    fwd_bytes = 4 * M * N * 2 + N * 2 + M * 4        # x, d in; h, y out
    bwd_bytes = 4 * M * N * 2 + N * 2 + M * 4        # dy, x, dres in; dx out
    sets = _rotated_sets(bwd_bytes)
    bufs = [tuple(torch.randn(M, N, device=dev, generator=g).to(torch.bfloat16) for _ in range(4))
            + (torch.rand(M, device=dev, generator=g) + 0.5, torch.empty(M, N, device=dev,
                                                                        dtype=torch.bfloat16))
            for _ in range(sets)]

    def fwd(b):
        x, d, h, y, rstd, _ = b
        _lib.call("qlora_add_rmsnorm_fwd", x.data_ptr(), d.data_ptr(), 2, N, N, w.data_ptr(), 2,
                  h.data_ptr(), N, y.data_ptr(), 2, N, rstd.data_ptr(), M, N, 1e-6,
                  _lib.stream_of(x))

    def bwd(b):
        dy, x, dres, _, rstd, dx = b
        _lib.call("qlora_rmsnorm_bwd_residual", dy.data_ptr(), 2, N, x.data_ptr(), 2, N,
                  w.data_ptr(), 2, rstd.data_ptr(), dres.data_ptr(), N, dx.data_ptr(), N, M, N,
                  _lib.stream_of(x))
    calls = 2 * sets
    _rate("add_rmsnorm_fwd_4096x3584", _graph_time(
        [lambda b=bufs[i % sets]: fwd(b) for i in range(calls)], torch, 3), fwd_bytes, res)
    _rate("rmsnorm_bwd_residual_4096x3584", _graph_time(
        [lambda b=bufs[i % sets]: bwd(b) for i in range(calls)], torch, 3), bwd_bytes, res)
    for name in ("add_rmsnorm_fwd_4096x3584", "rmsnorm_bwd_residual_4096x3584"):
        res[name]["rotated_sets"] = sets
    del bufs

    shapes = [(3584, 3584), (512, 3584), (512, 3584)]
    rows = sum(r for r, _ in shapes)
    items = [quant.quantize_nf4(torch.randn(sh, device=dev, generator=g) * 0.02, 64, True)
             for sh in shapes]
    nbytes = sum(nf4_algorithmic_bytes(r * c) for r, c in shapes)
    sets = _rotated_sets(nbytes, minimum=4)
    wsets = [(torch.empty(rows, N, device=dev, dtype=torch.bfloat16),
              torch.empty(N, rows, device=dev, dtype=torch.bfloat16)) for _ in range(sets)]
    offs = [0, 3584, 4096, 4608]

    def plain(i):
        wb = wsets[i % sets][0]
        nf4.dequantize_nf4_group(items, torch.bfloat16, [wb[offs[j]:offs[j + 1]] for j in range(3)])

    def trans(i):
        wt = wsets[i % sets][1]
        nf4.dequantize_nf4_t_group(items, torch.bfloat16,
                                   [wt[:, offs[j]:offs[j + 1]] for j in range(3)])
    _rate("nf4_dequant_group_qkv_7b", _graph_time([lambda i=i: plain(i) for i in range(2 * sets)],
                                                   torch, 3), nbytes, res)
    _rate("nf4_dequant_t_group_qkv_7b", _graph_time([lambda i=i: trans(i) for i in range(2 * sets)],
                                                     torch, 3), nbytes, res)
    del wsets, items

    n = 18944 * 3584
    wq = (torch.randn(n, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    packed = torch.empty(n // 2, dtype=torch.uint8, device=dev)
    nb = n // 64
    absmax = torch.empty(nb, dtype=torch.uint8, device=dev)
    absmax2 = torch.empty(_m.ceil(nb / 256), dtype=torch.float32, device=dev)
    offset = torch.empty((), dtype=torch.float32, device=dev)
    code, code2 = quant.nf4_code(dev), quant.dynamic_map(True).to(dev)
    ws, ws_bytes = _lib.workspace("qlora_nf4_quantize_workspace_size", n, 64, 1, device=dev)

    def qz():
        _lib.call("qlora_nf4_quantize", wq.data_ptr(), 2, n, 64, 1, 256, code.data_ptr(),
                  code2.data_ptr(), packed.data_ptr(), absmax.data_ptr(), absmax2.data_ptr(),
                  offset.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_of(wq))
    qbytes = 2 * n + n // 2 + nb + 4 * _m.ceil(nb / 256)
    _rate("nf4_quantize_18944x3584", _event_time(qz, torch), qbytes, res)
    del wq, packed, absmax, ws

    cfg = qlora_step.qwen2_config()
    H, I, KV = cfg.hidden_size, cfg.intermediate_size, cfg.num_key_value_heads * 128
    shapes = []
    for _ in range(cfg.num_hidden_layers):
        for out_f, in_f in ((H, H), (KV, H), (KV, H), (H, H), (I, H), (I, H), (H, I)):
            shapes += [(16, in_f), (out_f, 16)]
    tensors = [[torch.randn(sh, device=dev, generator=g) * 0.01 for _ in range(4)]
               for sh in shapes]
    for t in tensors:
        t[3].abs_()
    chunk = int(_lib.load().qlora_adamw_chunk_elems())
    table, first = [], 0
    for p_, g_, m_, v_ in tensors:
        table.append([p_.data_ptr(), g_.data_ptr(), m_.data_ptr(), v_.data_ptr(), p_.numel(), first])
        first += (p_.numel() + chunk - 1) // chunk
    table_d = torch.tensor(table, dtype=torch.int64).to(dev)
    values = sum(t[0].numel() for t in tensors)

    def adamw():
        _lib.call("qlora_adamw_fp32", table_d.data_ptr(), len(tensors), first, 1.0, 0.999, 0.1,
                  0.001, 1e-4, 0.05, 1e-8, _lib.stream_of(table_d))
    _rate("adamw_fp32_7b_adapters", _graph_time([adamw] * 10, torch, 3), 28 * values, res)
    res["adamw_fp32_7b_adapters"]["values"] = values


def bench_kernels(torch):
    """Device time per call and roofline fraction of the other kernels at their configs."""
    res = {}
    bench_rmsnorm(torch, res)
    bench_rope(torch, res)
    bench_swiglu(torch, res)
    bench_gemms(torch, res)
    bench_ce(torch, res)
    res["qwen25_7b_mlp_lora_4096tok"] = bench_mlp(torch)
    bench_next_rows(torch, res)
    return res


def bench_gemm_data(torch, res, reps=20, sets=3):
    """The NT GEMM at the 7B MLP's two shapes with the same schedule on different operand data:
    N(0,1) values, all zeros, small integers in [-2, 2] (few mantissa bits toggling) and
    NF4-like weights (16 levels times a per-64 scale) against N(0,1) activations. Identical
    instructions and memory traffic; a rate that moves with the data is a power/clock limit,
    and the all-zero rate is the schedule's ceiling on this part."""
    from hackathon_amd import gemm

    dev = "cuda"
    levels = torch.tensor([-1.0, -0.6962, -0.5251, -0.3949, -0.2844, -0.1848, -0.0911, 0.0,
                           0.0796, 0.1609, 0.2461, 0.3379, 0.4407, 0.5626, 0.7230, 1.0],
                          device=dev)
    for Mm, Nn, Kk in ((4096, 18944, 3584), (4096, 3584, 18944)):
        g = torch.Generator(device=dev).manual_seed(1)
        entry = {}
        for kind in ("randn", "zeros", "int", "nf4_weights"):
            bufs = []
            for _ in range(sets):
                if kind == "zeros":
                    a = torch.zeros(Mm, Kk, device=dev, dtype=torch.bfloat16)
                    b = torch.zeros(Nn, Kk, device=dev, dtype=torch.bfloat16)
                elif kind == "int":
                    a = torch.randint(-2, 3, (Mm, Kk), device=dev, generator=g).to(torch.bfloat16)
                    b = torch.randint(-2, 3, (Nn, Kk), device=dev, generator=g).to(torch.bfloat16)
                else:
                    a = torch.randn(Mm, Kk, device=dev, generator=g).to(torch.bfloat16)
                    if kind == "randn":
                        b = torch.randn(Nn, Kk, device=dev, generator=g).to(torch.bfloat16)
                    else:
                        idx = torch.randint(0, 16, (Nn, Kk), device=dev, generator=g)
                        sc = torch.rand(Nn, Kk // 64, 1, device=dev, generator=g) * 0.05 + 0.03
                        b = (levels[idx].view(Nn, Kk // 64, 64) * sc).view(Nn, Kk).to(torch.bfloat16)
                bufs.append((a, b, torch.empty(Mm, Nn, dtype=torch.bfloat16, device=dev)))
            fns = [(lambda bb=bufs[i % sets]: gemm.gemm_nt_cat(bb[0], bb[1], None, None, bb[2]))
                   for i in range(reps)]
            t = _graph_time(fns, torch, replays=3)
            fl = 2.0 * Mm * Nn * Kk
            entry[kind] = dict(us=round(t * 1e6, 1), tflops=round(fl / t / 1e12, 1))
            del bufs, fns
        res[f"gemm_data_{Mm}x{Nn}x{Kk}"] = entry
    # the matrix cores without global memory traffic (qlora_mfma_probe: the GEMM's 4 x 4
    # product pattern, one wave per SIMD; mode 0 fragments in registers, mode 1 read from LDS)
    # on the same kinds of data
    from hackathon_amd import _lib

    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(256 * n_cu, dtype=torch.float32, device=dev)
    src = torch.randn(2 << 19, device=dev).to(torch.bfloat16)  # 2 MiB for mode 2's loads
    iters = 2000
    for mode, name in ((0, "registers"), (1, "lds_fragments"), (2, "lds_fragments_dma"),
                       (3, "lds_fragments_vgpr_loads")):
        probe = {}
        for kind in ("randn", "zeros", "int"):
            g = torch.Generator(device=dev).manual_seed(2)
            n_el = 1024 * 8  # 1024 uint4 of 16-bit values
            if kind == "zeros":
                ops = torch.zeros(n_el, dtype=torch.bfloat16, device=dev)
            elif kind == "int":
                ops = torch.randint(-2, 3, (n_el,), device=dev, generator=g).to(torch.bfloat16)
            else:
                ops = torch.randn(n_el, device=dev, generator=g).to(torch.bfloat16)

            def run(o=ops, m=mode):
                _lib.call("qlora_mfma_probe", o.data_ptr(), _lib.tag(torch.bfloat16), m, iters,
                          n_cu, out.data_ptr(), src.data_ptr(), _lib.stream_of(out))

            t = _event_time(run, torch, calls=5, warm=2)
            fl = n_cu * 4 * (iters // 2 * 2 if mode >= 2 else iters) * 32 * 32768.0
            probe[kind] = dict(us=round(t * 1e6, 1), tflops=round(fl / t / 1e12, 1))
        res[f"mfma_probe_32x32x16_bf16_{name}"] = probe


def bench_dropout(torch, res, replays=10):
    """LoRA dropout at the 7B step's shapes (4096 rows, p = 0.05, bf16), per adapter group:
    forward, the dropout kernel plus lora_down for each adapter, the dropout kernel alone, and
    the one-pass qlora_lora_dropout_down with the dropped inputs stored and without them (bits
    and u only, as the step runs it; also without its K split); backward, the lora_A gradients
    as lora_wgrad over each stored dropped input against qlora_lora_wgrad_masked over x and the
    bits. Forward rates are Philox draws per second (one per input element and adapter)."""
    import ctypes

    from hackathon_amd import _lib, gemm, lora

    dt, p = torch.bfloat16, 0.05
    g = torch.Generator(device="cuda").manual_seed(0)
    for M, K, G in ((4096, 3584, 3), (4096, 3584, 2), (4096, 3584, 1), (4096, 18944, 1)):
        x = torch.randn(M, K, device="cuda", generator=g).to(dt)
        a16 = (0.1 * torch.randn(16 * G, K, device="cuda", generator=g)).to(dt)
        u = torch.empty(M, 64, device="cuda", dtype=dt)
        ut = gemm.lora_t_buffer(M, dt, "cuda", rows=16 * G)
        seeds = [1234 + i for i in range(G)]
        xds = [torch.empty(M, K, device="cuda", dtype=dt) for _ in range(G)]
        bitss = [lora.keep_bits_buffer(M, K, "cuda") for _ in range(G)]
        sa = (ctypes.c_uint64 * G)(*seeds)
        xp = (ctypes.c_void_p * G)(*[t.data_ptr() for t in xds])
        bp = (ctypes.c_void_p * G)(*[t.data_ptr() for t in bitss])
        ws, ws_bytes = _lib.workspace("qlora_lora_dropout_down_workspace_size", M, K, G,
                                      device="cuda")

        def per_adapter(down=True):
            for i in range(G):
                _lib.call("qlora_lora_dropout_scale_bits", x.data_ptr(), K, xds[i].data_ptr(), K,
                          bitss[i].data_ptr(), K, M, K, _lib.tag(dt), seeds[i], p, 1 / (1 - p),
                          _lib.stream_of(x))
                if down:
                    gemm.lora_down(xds[i], a16[16 * i:16 * i + 16], u[:, 16 * i:],
                                   out_t=ut[16 * i:16 * i + 16])

        def one_pass(xdp=xp, w=ws, nb=ws_bytes):
            _lib.call("qlora_lora_dropout_down", x.data_ptr(), K, a16.data_ptr(), K, M, K, G,
                      _lib.tag(dt), sa, p, 1 / (1 - p), xdp, K, bp, K, u.data_ptr(), 64, 64,
                      ut.data_ptr(), ut.stride(0), _lib.ptr(w), nb, _lib.stream_of(x))

        def wgrad_per_adapter():
            for i in range(G):
                gemm.lora_wgrad(ut[16 * i:16 * i + 16], xds[i], transposed=True)

        def wgrad_masked():
            gemm.lora_wgrad_masked(ut, x, bitss, p)

        draws = G * M * K
        entry = {}
        for name, fn in (("dropout_and_lora_down_per_adapter", per_adapter),
                         ("dropout_alone", lambda: per_adapter(False)),
                         ("one_pass_with_xd", one_pass),
                         ("one_pass", lambda: one_pass(None)),
                         ("one_pass_unsplit", lambda: one_pass(None, None, 0))):
            t = _graph_time([fn] * 4, torch, replays)
            entry[name] = dict(us=round(t * 1e6, 1), gdraws_per_s=round(draws / t / 1e9, 1))
        entry["splits"] = 1 if ws_bytes == 0 else ws_bytes // (M * 16 * G * 4)
        per_adapter()  # the stored dropped inputs and bits for the gradient timings
        for name, fn in (("lora_a_grad_per_adapter_on_xd", wgrad_per_adapter),
                         ("lora_a_grad_masked", wgrad_masked)):
            entry[name] = dict(us=round(_graph_time([fn] * 4, torch, replays) * 1e6, 1))
        res[f"dropout_down_{M}x{K}x{G}"] = entry
    # the down adapter's dropout inside the SwiGLU forward (h, its keep bits and u) against the
    # dropout-free kernel and against the SwiGLU kernel plus the one-pass dropout of h
    from hackathon_amd import swiglu

    M, n = 4096, 18944
    gu = torch.randn(M, 2 * n, device="cuda", generator=g).to(dt)
    a = (0.05 * torch.randn(16, n, device="cuda", generator=g)).to(dt)
    h = torch.empty(M, n, device="cuda", dtype=dt)
    u = torch.empty(M, 64, device="cuda", dtype=dt)
    ut = gemm.lora_t_buffer(M, dt, "cuda")
    entry = {}
    for name, fn in (
            ("swiglu_fwd_lora_down", lambda: swiglu.swiglu_fwd_lora_down(
                gu[:, :n], gu[:, n:], h, a, u, ut)),
            ("swiglu_fwd_lora_down_dropout", lambda: swiglu.swiglu_fwd_lora_down(
                gu[:, :n], gu[:, n:], h, a, u, ut, p=p, seed=99)),
            ("swiglu_rows_then_one_pass_dropout", lambda: (
                swiglu.swiglu_rows(gu[:, :n], gu[:, n:], h),
                lora.dropout_down(h, a, p, (99,), u, ut)))):
        entry[name] = dict(us=round(_graph_time([fn] * 4, torch, replays) * 1e6, 1))
    res[f"swiglu_down_dropout_{M}x{n}"] = entry


WORKLOADS = {
    "gemm_data": lambda torch, res: bench_gemm_data(torch, res),
    "rmsnorm": lambda torch, res: bench_rmsnorm(torch, res),
    "rope": lambda torch, res: bench_rope(torch, res),
    "swiglu": lambda torch, res: bench_swiglu(torch, res),
    "gemm": lambda torch, res: bench_gemms(torch, res),
    "ce": lambda torch, res: bench_ce(torch, res),
    "mlp": lambda torch, res: res.update(qwen25_7b_mlp_lora_4096tok=bench_mlp(torch)),
    "nf4_small": lambda torch, res: res.update(nf4_4864x896=bench_nf4_small(torch)),
    "next": lambda torch, res: bench_next_rows(torch, res),
    "dropout": lambda torch, res: bench_dropout(torch, res),
}


def calibration_copy(torch, mib=256):
    """One plain device-to-device copy of `mib` MiB (known bytes each way): the reference
    dispatch that scales rocprofv3's FETCH_SIZE / WRITE_SIZE to bytes in the same run."""
    src = torch.ones(mib * 2**19, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def bench_mlp(torch, tokens=4096, reps=3):
    """The Qwen2.5-7B MLP with NF4 bases and LoRA r=16 on gate/up/down, forward + backward at
    `tokens` tokens (gradients to the adapters and the input), patched and eager. Work: the
    three base projections forward and their dX backward, 2 x (3 x 2 T H I) FLOP, plus the
    rank-16 products, 6 T r (H + I) FLOP per projection (u, its share of y; du, its share of
    dX, dA, dB): 3.364 TFLOP at T = 4096."""
    from hackathon_amd import qlora_step

    cfg = qlora_step.qwen2_config(num_hidden_layers=1, vocab_size=1024)
    model = qlora_step.build_qlora_model(cfg, "cuda")
    mlp = model.model.layers[0].mlp
    H, I, r = cfg.hidden_size, cfg.intermediate_size, 16
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(1, tokens, H, device="cuda", generator=g).to(torch.bfloat16).requires_grad_()
    dy = torch.randn(1, tokens, H, device="cuda", generator=g).to(torch.bfloat16)
    params = qlora_step.lora_parameters(model)
    base = 2 * (3 * 2.0 * tokens * H * I)
    lora = 3 * 6.0 * tokens * r * (H + I)
    fl = base + lora

    def one():
        x.grad = None
        for p in params:
            p.grad = None
        mlp(x).backward(dy)

    def timed():
        one()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            one()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / reps

    qlora_step.patched_mode()
    t = timed()
    with qlora_step.eager_mode(model):
        t_e = timed()
    qlora_step.patched_mode()
    del model, mlp, x, dy, params
    return dict(ms=round(t * 1e3, 3), tflops=round(fl / t / 1e12, 1),
                frac_mfma=round(fl / t / 1e12 / BF16_PEAK_TFLOPS, 3), work_tflop=round(fl / 1e12, 3),
                eager_ms=round(t_e * 1e3, 3), speedup_vs_eager=round(t_e / t, 2))


# ---------------------------------------------------------------------------------------------
def bench_step(torch, steps, warmup, eager_steps=2, layers=None, batch=2, seq=2048,
               parity=True, dropout=0.0):
    """Qwen2.5-7B-shaped QLoRA step (28 layers unless `layers`), tokens/s patched and eager.
    With `dropout` > 0 every LoRA adapter drops its input with that probability (the
    reference's training regime, p = 0.05): the patched layers draw the mask from the package's
    Philox stream and eager from torch's RNG, so the step-0 losses differ by the masks."""
    from hackathon_amd import qlora_step

    over = {} if layers is None else {"num_hidden_layers": layers}
    cfg = qlora_step.qwen2_config(**over)
    t0 = time.perf_counter()
    model = qlora_step.build_qlora_model(cfg, "cuda", dropout=dropout)
    torch.cuda.synchronize()
    log(f"[bench] model built in {time.perf_counter() - t0:.1f} s")
    ids, labels = qlora_step.make_batch(batch, seq, cfg.vocab_size)
    tokens = batch * seq

    def run(step, k, w):
        for _ in range(w):
            step(ids, labels)
        torch.cuda.synchronize()
        t = time.perf_counter()
        loss = None
        for _ in range(k):
            loss = step(ids, labels)
        torch.cuda.synchronize()
        return (time.perf_counter() - t) / k, float(loss)

    # loss parity at identical parameters, before any optimizer step
    qlora_step.patched_mode()
    step = qlora_step.QLoRAStep(model, fused_head=True)
    loss_p0 = loss_e0 = float("nan")
    if parity:
        loss_p0 = float(step.forward_backward(ids, labels))
        model.zero_grad(set_to_none=True)
        with qlora_step.eager_mode(model):
            loss_e0 = float(qlora_step.QLoRAStep(model, fused_head=False).forward_backward(ids,
                                                                                         labels))
        model.zero_grad(set_to_none=True)
        qlora_step.patched_mode()
        log(f"[bench] step-0 loss patched {loss_p0:.6f} eager {loss_e0:.6f}")
    torch.cuda.reset_peak_memory_stats()  # the patched steps' own peak, not the parity runs'
    t_p, loss_p = run(step, steps, warmup)
    log(f"[bench] patched step {t_p * 1e3:.1f} ms loss {loss_p:.4f}")
    peak_p = torch.cuda.max_memory_allocated() / 2**30
    torch.cuda.reset_peak_memory_stats()
    out = dict(tokens_per_step=tokens, ms_per_step=round(t_p * 1e3, 1),
               tokens_per_s=round(tokens / t_p, 1), loss=round(loss_p, 5),
               step0_loss_patched=round(loss_p0, 6), step0_loss_eager=round(loss_e0, 6),
               step0_loss_rel_diff=round(abs(loss_p0 - loss_e0) / abs(loss_e0), 7),
               peak_mem_gib=round(peak_p, 1), layers=cfg.num_hidden_layers,
               lora_dropout=dropout)
    if eager_steps:
        with qlora_step.eager_mode(model):
            step_e = qlora_step.QLoRAStep(model, fused_head=False)
            t_e, loss_e = run(step_e, eager_steps, 1)
        log(f"[bench] eager step {t_e * 1e3:.1f} ms loss {loss_e:.4f}")
        out.update(eager_ms_per_step=round(t_e * 1e3, 1), eager_tokens_per_s=round(tokens / t_e, 1),
                   speedup_vs_eager=round(t_e / t_p, 3),
                   eager_peak_mem_gib=round(torch.cuda.max_memory_allocated() / 2**30, 1))
        qlora_step.patched_mode()
    del model, step
    return out


# ---------------------------------------------------------------------------------------------
def _trace_category(name):
    """Step-breakdown category of a kernel name from a rocprofv3 kernel trace."""
    table = (("attn_fwd_kernel", "attention fwd (flash)"), ("attn_bwd_dkdv", "attention dK/dV"),
             ("attn_bwd_dq", "attention dQ (with Delta)"),
             ("attn_bwd_reduce", "attention dK/dV head sum"),
             ("gemm_nt_kernel", "NT GEMM (incl. the LoRA K segment)"),
             ("splitk_reduce", "GEMM split-K reduce"), ("gemm_mfma_kernel", "GEMM (general)"),
             ("lora_down", "lora_down (+reduce)"), ("lora_wgrad", "lora_wgrad (+reduce)"),
             ("lora_pack", "lora_pack"), ("nf4_dequant_t", "NF4 dequant (transposed)"),
             ("nf4_dequant", "NF4 dequant"), ("swiglu", "SwiGLU"), ("rmsnorm", "RMSNorm"),
             ("rope", "RoPE"), ("ce_rows", "CE rows"), ("transpose16", "transpose"),
             ("Cijk", "hipBLASLt"), ("multi_tensor_apply", "torch AdamW (foreach)"),
             ("adamw_multi_fp32", "AdamW (fused)"),
             ("dropout_down_kernel", "LoRA dropout + down-projection (mask, bits, u)"),
             ("dropout_bits_kernel", "LoRA dropout (Philox mask + bits)"),
             ("dropout_scale_kernel", "LoRA dropout / cast"),
             ("up_masked_add", "LoRA dropout backward (masked rank-16 add)"),
             ("scaled_add", "LoRA scaled add"),
             ("CUDAFunctor_add", "torch add"))
    for key, cat in table:
        if key in name:
            return cat
    return "torch other"


def trace_summary(path):
    """Per-step kernel time of the patched QLoRA step from a rocprofv3 --kernel-trace CSV.
    Steps are delimited by the embedding gather (one vectorized_gather_kernel per step); the
    table is for the last complete step."""
    import collections
    import csv

    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if "vectorized_gather_kernel" in r["Kernel_Name"]]
    if len(marks) < 2:
        raise SystemExit("trace holds fewer than two steps")
    a, b = marks[-2], marks[-1]
    agg, cnt = collections.Counter(), collections.Counter()
    for r in rows[a:b]:
        c = _trace_category(r["Kernel_Name"])
        agg[c] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6
        cnt[c] += 1
    span = (int(rows[b]["Start_Timestamp"]) - int(rows[a]["Start_Timestamp"])) / 1e6
    total = sum(agg.values())
    print(f"steps in trace: {len(marks)}; last complete step: wall {span:.1f} ms, "
          f"kernel time {total:.1f} ms")
    print("| category | launches | ms per step | % of kernel time |\n|---|---|---|---|")
    for k, v in agg.most_common():
        print(f"| {k} | {cnt[k]} | {v:.2f} | {100 * v / total:.1f} |")


def _short_kernel(name, width=64):
    """Kernel name without its argument list, clipped for a table."""
    name = name.replace("(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for i, ch in enumerate(name):
        depth += (ch == "<") - (ch == ">")
        if ch == "(" and depth == 0:
            name = name[:i]
            break
    return name if len(name) <= width else name[: width - 3] + "..."


def pmc_summary(counter_csv):
    """Per kernel of a rocprofv3 --pmc counter_collection.csv: dispatches and, for each counter,
    the mean over dispatches of its value (summed over the counter's hardware instances by
    rocprofv3), as a markdown table."""
    import collections
    import csv

    sums = collections.defaultdict(lambda: collections.defaultdict(float))
    dispatches = collections.defaultdict(set)
    counters = set()
    for r in csv.DictReader(open(counter_csv)):
        name = r["Kernel_Name"].replace("(anonymous namespace)::", "").replace("void ", "")
        name = name.split("(")[0][:48]
        sums[name][r["Counter_Name"]] += float(r["Counter_Value"])
        dispatches[name].add(r["Dispatch_Id"])
        counters.add(r["Counter_Name"])
    cols = sorted(counters)
    print("| kernel | dispatches | " + " | ".join(cols) + " |")
    print("|---|---|" + "---|" * len(cols))
    for name in sorted(sums):
        n = len(dispatches[name])
        print(f"| `{name}` | {n} | " + " | ".join(f"{sums[name][c] / n:.4g}" for c in cols) + " |")


def profile_summary(trace_csv, fetch_csv=None, write_csv=None, copy_mib=256):
    """Markdown table of a rocprofv3 run: per (kernel, grid size) the dispatch count and the
    average / min / max duration from the kernel trace; with the two PMC passes of the same
    command, FETCH_SIZE and WRITE_SIZE per dispatch scaled to bytes by the run's calibration
    copy (the largest __amd_rocclr_copyBuffer dispatch, `copy_mib` MiB each way)."""
    import collections
    import csv

    def key(name, grid):
        return (_short_kernel(name), int(grid))

    durs = collections.defaultdict(list)
    for r in csv.DictReader(open(trace_csv)):
        grid = int(r["Grid_Size_X"]) * int(r.get("Grid_Size_Y") or 1) * int(r.get("Grid_Size_Z") or 1)
        durs[key(r["Kernel_Name"], grid)].append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)

    def counters(path, counter):
        per, calib = collections.defaultdict(list), None
        if path is None:
            return per, None
        vals = collections.defaultdict(float)
        names = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] != counter:
                continue
            d = r["Dispatch_Id"]
            vals[d] += float(r["Counter_Value"])
            names[d] = (r["Kernel_Name"], r["Grid_Size"])
        copies = [v for d, v in vals.items() if "copyBuffer" in names[d][0]]
        if copies:
            calib = copy_mib * 1024 / max(copies)
        for d, v in vals.items():
            per[key(*names[d])].append(v * 1024 * (calib or 1.0))
        return per, calib

    fetch, fcal = counters(fetch_csv, "FETCH_SIZE")
    write, wcal = counters(write_csv, "WRITE_SIZE")
    total = sum(sum(v) for v in durs.values())
    head = "| kernel | grid | calls | avg us | min us | max us | % time |"
    sep = "|---|---|---|---|---|---|---|"
    if fetch_csv:
        head += " fetch MB/call | write MB/call |"
        sep += "---|---|"
    print(head)
    print(sep)
    for k, v in sorted(durs.items(), key=lambda kv: -sum(kv[1])):
        row = (f"| `{k[0]}` | {k[1]} | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | "
               f"{max(v):.2f} | {100 * sum(v) / total:.1f} |")
        if fetch_csv:
            f, w = fetch.get(k), write.get(k)
            row += (f" {sum(f) / len(f) / 1e6:.2f} |" if f else " - |")
            row += (f" {sum(w) / len(w) / 1e6:.2f} |" if w else " - |")
        print(row)
    if fetch_csv:
        print(f"\ncalibration ({copy_mib} MiB device copy in the same run): FETCH_SIZE x"
              f"{fcal if fcal is None else round(fcal, 4)}, WRITE_SIZE x"
              f"{wcal if wcal is None else round(wcal, 4)}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sets", type=int, default=4, help="rotated buffer sets for the dequant")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-step", action="store_true", help="skip the 7B QLoRA step")
    ap.add_argument("--no-kernels", action="store_true", help="skip the per-kernel table")
    ap.add_argument("--no-cpu-configs", action="store_true",
                    help="skip the host CPU baselines of the other configs")
    ap.add_argument("--step-steps", type=int, default=5)
    ap.add_argument("--no-dropout-step", action="store_true",
                    help="skip the step with LoRA dropout 0.05")
    ap.add_argument("--step-dropout", type=float, default=0.0,
                    help="LoRA dropout of the main step entry (default 0; with it set, the "
                         "separate dropout-0.05 entry is not run)")
    ap.add_argument("--step-layers", type=int, default=None)
    ap.add_argument("--eager-steps", type=int, default=2,
                    help="timed steps of the eager baseline (0: skip it and the parity check)")
    ap.add_argument("--nf4-only", action="store_true", help="only the dequant (for profiling)")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run a 256 MiB device copy (counter calibration) and eight eager dequant "
                         "launches, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="print the per-step kernel table of a rocprofv3 kernel trace and exit")
    ap.add_argument("--workload", choices=sorted(WORKLOADS),
                    help="run one workload of the kernel table alone, after a 256 MiB calibration "
                         "copy, and print its JSON (for rocprofv3 kernel-trace and PMC passes)")
    ap.add_argument("--profile-summary", nargs="+", metavar="CSV",
                    help="per-kernel table from a rocprofv3 kernel_trace.csv, optionally followed "
                         "by FETCH_SIZE and WRITE_SIZE counter_collection.csv files of the same "
                         "command (calibrated by its copy kernel); prints markdown and exits")
    ap.add_argument("--pmc-summary", metavar="CSV",
                    help="per-kernel mean of every counter in a rocprofv3 --pmc "
                         "counter_collection.csv; prints markdown and exits")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.profile_summary:
        profile_summary(*args.profile_summary)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): the kernels work on one "
              f"GPU's share and there is no multi-GPU path", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from hackathon_amd import _lib

    _lib.load()  # fail loudly if the kernel library is not built
    shape = (18944, 3584)
    if args.pmc_probe:
        pmc_probe(torch, shape)
        return
    if args.workload:
        calibration_copy(torch)
        res = {}
        WORKLOADS[args.workload](torch, res)
        torch.cuda.synchronize()
        print(json.dumps({"workload": args.workload, **res}), flush=True)
        return
    torch.cuda.synchronize()
    r = bench_nf4(torch, shape, args.steps, args.warmup, args.sets)
    log(f"[bench] nf4 {shape}: {r['sec_per_call'] * 1e6:.2f} us/call, {r['gbs']:.0f} GB/s")
    line = {
        "metric": METRIC, "value": round(r["gbs"], 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(r["sec_per_call"] * 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u8->bf16 (fp32 math)",
        "data": "synthetic: N(0,0.02) weights quantised to NF4 in-process",
        "config": {"workload": "nf4_dequant 18944x3584 (Qwen2.5-7B gate_proj) blocksize 64, "
                               "double-quant absmax blocksize 256, bf16 out",
                   "weights": r["n"], "rotated_sets": args.sets, "timing": "HIP graph of "
                   f"{args.steps} launches, HIP events on the launch stream"},
        "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": _measured_traffic(),
                     "traffic_source": "stored: profiles/nf4_dequant_traffic.json, rocprofv3 "
                                       "--pmc FETCH_SIZE and WRITE_SIZE passes over bench.py "
                                       "--pmc-probe, scaled by a 256 MiB copy in the same run"},
    }
    if args.nf4_only:
        print(json.dumps(line), flush=True)
        return
    hp = hbm_practical(torch)
    hp["dequant_frac_of_write"] = round(r["gbs"] / hp["write_fill_gbs"], 4)
    line["hbm_practical"] = hp
    log(f"[bench] HBM practical: {json.dumps(hp)}")
    r1 = line["nf4_4864x896"] = bench_nf4_small(torch, max(args.steps, 200), args.warmup)
    log(f"[bench] nf4 4864x896: {r1['us']:.2f} us/call, {r1['gbs']:.0f} GB/s; launch floor "
        f"{r1['launch_floor_us']:.2f} us, {r1['above_floor_gbs']} GB/s above it; a copy / fill "
        f"of the same bytes {r1['copy_same_bytes_us']:.2f} / {r1['fill_same_bytes_us']:.2f} us")
    if not args.no_kernels:
        line["kernels"] = bench_kernels(torch)
        log(f"[bench] kernels: {json.dumps(line['kernels'])}")
    if not args.no_step:
        line["qlora_step"] = bench_step(torch, args.step_steps, 2, eager_steps=args.eager_steps,
                                        layers=args.step_layers, parity=args.eager_steps > 0,
                                        dropout=args.step_dropout)
        if not args.no_dropout_step and args.step_dropout == 0:
            torch.cuda.empty_cache()
            line["qlora_step_dropout"] = bench_step(
                torch, args.step_steps, 2, eager_steps=args.eager_steps, layers=args.step_layers,
                parity=args.eager_steps > 0, dropout=0.05)
    line["cpu_baseline"] = cpu_baseline_nf4(args.cpu_seconds)
    line["cpu_baseline"]["host_cpu"] = _cpu_model()
    line["cpu_baseline_c_1thread"] = cpu_baseline_nf4_c(min(args.cpu_seconds, 5.0))
    if not args.no_cpu_configs:
        t0 = time.perf_counter()
        line["cpu_baselines"] = cpu_baselines(torch)
        log(f"[bench] cpu baselines in {time.perf_counter() - t0:.0f} s: "
            f"{json.dumps(line['cpu_baselines'])}")
    print(json.dumps(line), flush=True)


def hbm_practical(torch, mib=1024, reps=20):
    """The box's practical HBM rates for the same kind of traffic, measured beside the
    dequant: a 1 GiB fill (pure write, the dequant's 79% share) and a 1 GiB device copy
    (read + write), HIP events on the current stream."""
    n = mib * 2**20
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3

    write = n / timed(lambda: b.fill_(7)) / 1e9
    copy = 2 * n / timed(lambda: b.copy_(a)) / 1e9
    del a, b
    return {"write_fill_gbs": round(write, 1), "copy_rw_gbs": round(copy, 1),
            "buffer_mib": mib}


def pmc_probe(torch, shape, sets=4, launches=8):
    """Kernels for the HBM-traffic counter passes: one plain device-to-device copy of
    256 MiB (hipMemcpyAsync, known bytes: it calibrates FETCH_SIZE / WRITE_SIZE), then
    `launches` eager dequants of the 7B gate weight rotating over `sets` buffer sets."""
    from hackathon_amd import nf4, quant

    src = torch.ones(128 * 2**20, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    g = torch.Generator(device="cuda").manual_seed(0)
    w = torch.randn(shape, device="cuda", generator=g) * 0.02
    packed, st = quant.quantize_nf4(w, 64, compress_statistics=True)
    del w
    bufs = [(packed.clone(), torch.empty(shape, dtype=torch.bfloat16, device="cuda"))
            for _ in range(sets)]
    torch.cuda.synchronize()
    for i in range(launches):
        p, o = bufs[i % sets]
        nf4.dequantize_nf4(p, st, torch.bfloat16, out=o)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_probe": True, "copy_bytes": 2 * 128 * 2**20,
                      "dequant_alg_bytes": nf4_algorithmic_bytes(shape[0] * shape[1]),
                      "dequant_launches": launches}), flush=True)


def _measured_traffic():
    """HBM bytes per dequant launch from the committed rocprofv3 PMC summary, if present."""
    p = ROOT / "profiles" / "nf4_dequant_traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("bytes_per_launch")
        except (ValueError, OSError):
            return None
    return None


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip() + f" ({os.cpu_count()} logical cpus)"
    except OSError:
        pass
    return None


if __name__ == "__main__":
    main()
