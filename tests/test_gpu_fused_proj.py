"""The fused q/k/v (+ RoPE) and gate/up (+ SwiGLU) projections against the same layers run one
by one (each its own LoraNF4Linear, then HipRoPE / SwiGLU, gradients summed by autograd).

Both compute every sum in fp32 from the same bf16 operands; they differ in the order of the fp32
accumulation (split-K of the narrow k/v outputs, one dX GEMM instead of three added in bf16),
so outputs agree to bf16 rounding and gradients to a small relative error (tolerances below).
With LoRA dropout both paths draw the same seeds (the seed stream restarted before each), so
they drop the same elements and agree to the same tolerances.
"""

import pytest
import torch

import hackathon_amd
from hackathon_amd import fused_proj, lora, qlora_step, rope, swiglu

pytestmark = pytest.mark.gpu


def _model(seed=0, dropout=0.0):
    cfg = qlora_step.qwen2_config(hidden_size=512, intermediate_size=1024, num_hidden_layers=1,
                                  num_attention_heads=4, num_key_value_heads=2, vocab_size=1000)
    return cfg, qlora_step.build_qlora_model(cfg, "cuda", seed=seed, dropout=dropout)


def _reseed(seed):
    """Restart the adapters' dropout seed stream, so two runs draw the same masks."""
    lora._Seeds.gen = torch.Generator().manual_seed(seed)


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-30)).item()


def _params(layers):
    out = []
    for layer in layers:
        out += [layer.lora_A["default"].weight, layer.lora_B["default"].weight]
    return out


def _zero(params, x):
    for p in params:
        p.grad = None
    x.grad = None


@pytest.mark.parametrize("seq", [64, 200])
def test_qkv_rope_matches_separate_layers(seq):
    print(f"fused qkv seq={seq}", flush=True)
    cfg, model = _model()
    attn = model.model.layers[0].self_attn
    layers = (attn.q_proj, attn.k_proj, attn.v_proj)
    params = _params(layers)
    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(2, seq, 512, device="cuda", generator=g).to(torch.bfloat16).requires_grad_()
    pos = torch.arange(seq, device="cuda")[None]
    cos, sin = model.model.rotary_emb(x, pos)
    hq, hk, d = 4, 2, 128
    wq = torch.randn(2, hq, seq, d, device="cuda", generator=g).to(torch.bfloat16)
    wk = torch.randn(2, hk, seq, d, device="cuda", generator=g).to(torch.bfloat16)
    wv = torch.randn(2, hk, seq, d, device="cuda", generator=g).to(torch.bfloat16)

    def loss_of(q, k, v):
        return (q.float() * wq).sum() + (k.float() * wk).sum() + (v.float() * wv).sum()

    # one by one
    q = attn.q_proj(x).view(2, seq, hq, d).transpose(1, 2)
    k = attn.k_proj(x).view(2, seq, hk, d).transpose(1, 2)
    v = attn.v_proj(x).view(2, seq, hk, d).transpose(1, 2)
    q, k = rope.HipRoPE.apply(q, k, cos, sin)
    loss_of(q, k, v).backward()
    ref = [t.detach().clone() for t in (q, k, v)]
    ref_g = [x.grad.clone()] + [p.grad.clone() for p in params]
    _zero(params, x)

    specs, ab = fused_proj._group(layers, x)
    q2, k2, v2 = fused_proj.QKVRoPE.apply(x, cos, sin, hq, hk, tuple(specs), None, *ab)
    loss_of(q2, k2, v2).backward()
    for a, b in zip((q2, k2, v2), ref):
        assert a.shape == b.shape
        assert _rel(a, b) < 4e-3
    got_g = [x.grad] + [p.grad for p in params]
    for name, a, b in zip(["x", "Aq", "Bq", "Ak", "Bk", "Av", "Bv"], got_g, ref_g):
        assert a is not None and a.dtype == b.dtype, name
        assert _rel(a, b) < 1e-2, (name, _rel(a, b))


@pytest.mark.parametrize("seq", [96, 37])
def test_gate_up_swiglu_matches_separate_layers(seq):
    """seq 37: 74 token rows, so the fused SwiGLU backward's last 32-row block is ragged."""
    print(f"fused gate/up seq={seq}", flush=True)
    cfg, model = _model()
    mlp = model.model.layers[0].mlp
    layers = (mlp.gate_proj, mlp.up_proj)
    params = _params(layers)
    g = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn(2, seq, 512, device="cuda", generator=g).to(torch.bfloat16).requires_grad_()
    w = torch.randn(2, seq, 1024, device="cuda", generator=g).to(torch.bfloat16)

    h = swiglu.swiglu(mlp.gate_proj(x), mlp.up_proj(x))
    (h.float() * w).sum().backward()
    ref = h.detach().clone()
    ref_g = [x.grad.clone()] + [p.grad.clone() for p in params]
    _zero(params, x)

    specs, ab = fused_proj._group(layers, x)
    h2 = fused_proj.GateUpSwiGLU.apply(x, tuple(specs), None, *ab)
    (h2.float() * w).sum().backward()
    assert h2.shape == ref.shape and _rel(h2, ref) < 4e-3
    got_g = [x.grad] + [p.grad for p in params]
    for name, a, b in zip(["x", "Ag", "Bg", "Au", "Bu"], got_g, ref_g):
        assert _rel(a, b) < 1e-2, (name, _rel(a, b))


@pytest.mark.parametrize("seq", [96, 37])
def test_lora_mlp_matches_separate_layers(seq):
    """The whole 4-bit LoRA MLP as one autograd function (the down adapter's products on h
    fused into the SwiGLU kernels, h not kept) against gate, up and down run one by one:
    output, input gradient and all six adapter gradients."""
    print(f"fused LoRA MLP seq={seq}", flush=True)
    cfg, model = _model()
    mlp = model.model.layers[0].mlp
    layers = (mlp.gate_proj, mlp.up_proj, mlp.down_proj)
    params = _params(layers)
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(2, seq, 512, device="cuda", generator=g).to(torch.bfloat16).requires_grad_()
    w = torch.randn(2, seq, 512, device="cuda", generator=g).to(torch.bfloat16)

    out = mlp.down_proj(swiglu.swiglu(mlp.gate_proj(x), mlp.up_proj(x)))
    (out.float() * w).sum().backward()
    ref = out.detach().clone()
    ref_g = [x.grad.clone()] + [p.grad.clone() for p in params]
    _zero(params, x)

    specs, ab = fused_proj._group(layers[:2], x)
    dspec, a_d, b_d = fused_proj.lora_spec(mlp.down_proj, x)
    out2 = fused_proj.LoraMLP.apply(x, tuple(specs), dspec, None, None, *ab, a_d, b_d)
    (out2.float() * w).sum().backward()
    assert out2.shape == ref.shape and _rel(out2, ref) < 4e-3
    got_g = [x.grad] + [p.grad for p in params]
    for name, a, b in zip(["x", "Ag", "Bg", "Au", "Bu", "Ad", "Bd"], got_g, ref_g):
        assert _rel(a, b) < 1e-2, (name, _rel(a, b))
    assert fused_proj.fused_mlp(mlp, x) is not None  # the patched MLP takes this path


def test_lora_mlp_partial_grads_and_no_grad():
    """LoraMLP with the down adapter frozen returns no gradient for it and the same gradients
    for the others as with it trainable; under no_grad it gives the same output."""
    print("fused LoRA MLP, frozen down adapter", flush=True)
    cfg, model = _model(seed=1)
    mlp = model.model.layers[0].mlp
    g = torch.Generator(device="cuda").manual_seed(6)
    x = torch.randn(2, 64, 512, device="cuda", generator=g).to(torch.bfloat16).requires_grad_()
    w = torch.randn(2, 64, 512, device="cuda", generator=g).to(torch.bfloat16)
    specs, ab = fused_proj._group((mlp.gate_proj, mlp.up_proj), x)
    dspec, a_d, b_d = fused_proj.lora_spec(mlp.down_proj, x)
    out = fused_proj.LoraMLP.apply(x, tuple(specs), dspec, None, None, *ab, a_d, b_d)
    (out.float() * w).sum().backward()
    ref = [x.grad.clone()] + [t.grad.clone() for t in ab]
    with torch.no_grad():
        out0 = fused_proj.LoraMLP.apply(x, tuple(specs), dspec, None, None, *ab, a_d, b_d)
    assert torch.equal(out0, out)
    x.grad = None
    for t in ab:
        t.grad = None
    a_d.grad = b_d.grad = None
    a_d.requires_grad_(False)
    b_d.requires_grad_(False)
    try:
        out2 = fused_proj.LoraMLP.apply(x, tuple(specs), dspec, None, None, *ab, a_d, b_d)
        (out2.float() * w).sum().backward()
        assert a_d.grad is None and b_d.grad is None
        got = [x.grad] + [t.grad for t in ab]
        for a, b in zip(got, ref):
            assert torch.equal(a, b)
    finally:
        a_d.requires_grad_(True)
        b_d.requires_grad_(True)


@pytest.mark.parametrize("seq", [64, 37])
def test_qkv_rope_with_dropout_matches_separate_layers(seq):
    """LoRA dropout 0.05 on q, k and v: the group draws each adapter's own mask from the seed
    the layer one by one would draw (the same seed stream, in projection order), so the two
    paths drop the same elements; outputs and all gradients agree as without dropout. A run on
    other seeds gives other outputs (the masks are applied)."""
    print(f"fused qkv with dropout seq={seq}", flush=True)
    cfg, model = _model(dropout=0.05)
    attn = model.model.layers[0].self_attn
    layers = (attn.q_proj, attn.k_proj, attn.v_proj)
    params = _params(layers)
    g = torch.Generator(device="cuda").manual_seed(8)
    x = torch.randn(2, seq, 512, device="cuda", generator=g).to(torch.bfloat16).requires_grad_()
    pos = torch.arange(seq, device="cuda")[None]
    cos, sin = model.model.rotary_emb(x, pos)
    hq, hk, d = 4, 2, 128
    w = [torch.randn(2, h, seq, d, device="cuda", generator=g).to(torch.bfloat16)
         for h in (hq, hk, hk)]

    def loss_of(*qkv):
        return sum((t.float() * wt).sum() for t, wt in zip(qkv, w))

    _reseed(5)
    q = attn.q_proj(x).view(2, seq, hq, d).transpose(1, 2)
    k = attn.k_proj(x).view(2, seq, hk, d).transpose(1, 2)
    v = attn.v_proj(x).view(2, seq, hk, d).transpose(1, 2)
    q, k = rope.HipRoPE.apply(q, k, cos, sin)
    loss_of(q, k, v).backward()
    ref = [t.detach().clone() for t in (q, k, v)]
    ref_g = [x.grad.clone()] + [p.grad.clone() for p in params]
    _zero(params, x)

    specs, ab = fused_proj._group(layers, x)
    assert [s.p for s in specs] == [0.05] * 3
    _reseed(5)
    q2, k2, v2 = fused_proj.QKVRoPE.apply(x, cos, sin, hq, hk, tuple(specs),
                                          fused_proj._seeds(specs), *ab)
    loss_of(q2, k2, v2).backward()
    for a, b in zip((q2, k2, v2), ref):
        assert _rel(a, b) < 4e-3
    got_g = [x.grad] + [p.grad for p in params]
    for name, a, b in zip(["x", "Aq", "Bq", "Ak", "Bk", "Av", "Bv"], got_g, ref_g):
        assert a is not None and a.dtype == b.dtype, name
        assert _rel(a, b) < 1e-2, (name, _rel(a, b))
    _reseed(6)
    with torch.no_grad():
        q3, _, _ = fused_proj.QKVRoPE.apply(x, cos, sin, hq, hk, tuple(specs),
                                            fused_proj._seeds(specs), *ab)
    assert _rel(q3, ref[0]) > 1e-3


@pytest.mark.parametrize("seq", [96, 37])
def test_gate_up_swiglu_with_dropout_matches_separate_layers(seq):
    print(f"fused gate/up with dropout seq={seq}", flush=True)
    cfg, model = _model(dropout=0.05)
    mlp = model.model.layers[0].mlp
    layers = (mlp.gate_proj, mlp.up_proj)
    params = _params(layers)
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn(2, seq, 512, device="cuda", generator=g).to(torch.bfloat16).requires_grad_()
    w = torch.randn(2, seq, 1024, device="cuda", generator=g).to(torch.bfloat16)

    _reseed(3)
    h = swiglu.swiglu(mlp.gate_proj(x), mlp.up_proj(x))
    (h.float() * w).sum().backward()
    ref = h.detach().clone()
    ref_g = [x.grad.clone()] + [p.grad.clone() for p in params]
    _zero(params, x)

    specs, ab = fused_proj._group(layers, x)
    _reseed(3)
    h2 = fused_proj.GateUpSwiGLU.apply(x, tuple(specs), fused_proj._seeds(specs), *ab)
    (h2.float() * w).sum().backward()
    assert _rel(h2, ref) < 4e-3
    got_g = [x.grad] + [p.grad for p in params]
    for name, a, b in zip(["x", "Ag", "Bg", "Au", "Bu"], got_g, ref_g):
        assert _rel(a, b) < 1e-2, (name, _rel(a, b))


@pytest.mark.parametrize("seq", [96, 37])
def test_lora_mlp_with_dropout_matches_separate_layers(seq):
    """LoRA dropout 0.05 on gate, up and down: the fused LoRA MLP (the down adapter's mask of h
    drawn in the SwiGLU forward kernel, kept as bits, applied again to the recomputed h in the
    backward kernel) against gate, up and down run one by one with the same seeds: output,
    input gradient and all six adapter gradients, at the tolerances without dropout."""
    print(f"fused LoRA MLP with dropout seq={seq}", flush=True)
    cfg, model = _model(dropout=0.05)
    mlp = model.model.layers[0].mlp
    layers = (mlp.gate_proj, mlp.up_proj, mlp.down_proj)
    params = _params(layers)
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(2, seq, 512, device="cuda", generator=g).to(torch.bfloat16).requires_grad_()
    w = torch.randn(2, seq, 512, device="cuda", generator=g).to(torch.bfloat16)

    _reseed(5)
    out = mlp.down_proj(swiglu.swiglu(mlp.gate_proj(x), mlp.up_proj(x)))
    (out.float() * w).sum().backward()
    ref = out.detach().clone()
    ref_g = [x.grad.clone()] + [p.grad.clone() for p in params]
    _zero(params, x)

    specs, ab = fused_proj._group(layers[:2], x)
    dspec, a_d, b_d = fused_proj.lora_spec(mlp.down_proj, x)
    assert specs[0].p == dspec.p == 0.05
    _reseed(5)
    seeds = fused_proj._seeds(specs) + (lora._Seeds.next(),)
    out2 = fused_proj.LoraMLP.apply(x, tuple(specs), dspec, seeds, None, *ab, a_d, b_d)
    (out2.float() * w).sum().backward()
    assert out2.shape == ref.shape and _rel(out2, ref) < 4e-3
    got_g = [x.grad] + [p.grad for p in params]
    for name, a, b in zip(["x", "Ag", "Bg", "Au", "Bu", "Ad", "Bd"], got_g, ref_g):
        assert _rel(a, b) < 1e-2, (name, _rel(a, b))
    # another down seed drops other elements of h: the output moves
    _reseed(5)
    seeds = fused_proj._seeds(specs) + (lora._Seeds.next() + 1,)
    with torch.no_grad():
        out3 = fused_proj.LoraMLP.apply(x, tuple(specs), dspec, seeds, None, *ab, a_d, b_d)
    assert _rel(out3, ref) > 1e-4


def test_decoder_layer_with_dropout_takes_the_groups(monkeypatch):
    """With dropout the patched layer runs q/k/v as a group and the MLP as the fused LoRA MLP
    (gate/up as a group, the down adapter's mask of h in the SwiGLU kernels)."""
    print("fused routing with dropout", flush=True)
    cfg, model = _model(dropout=0.05)
    hackathon_amd.apply()
    calls = {"qkv": 0, "gate_up": 0, "mlp": 0}
    orig = {n: c.apply for n, c in (("qkv", fused_proj.QKVRoPE),
                                     ("gate_up", fused_proj.GateUpSwiGLU),
                                     ("mlp", fused_proj.LoraMLP))}
    for name, cls in (("qkv", fused_proj.QKVRoPE), ("gate_up", fused_proj.GateUpSwiGLU),
                      ("mlp", fused_proj.LoraMLP)):
        def counted(*a, _name=name):
            calls[_name] += 1
            return orig[_name](*a)

        monkeypatch.setattr(cls, "apply", counted)
    ids = torch.randint(0, 1000, (2, 64), device="cuda")
    out = model(input_ids=ids, labels=ids, use_cache=False)
    out.loss.backward()
    assert calls == {"qkv": 1, "gate_up": 0, "mlp": 1}
    assert all(p.grad is not None and torch.isfinite(p.grad).all()
               for p in qlora_step.lora_parameters(model))


def test_swiglu_rows_match_the_contiguous_kernels():
    print("swiglu rows", flush=True)
    g = torch.Generator(device="cuda").manual_seed(3)
    y = torch.randn(37, 2 * 264, device="cuda", generator=g).to(torch.bfloat16)
    gate, up = y[:, :264], y[:, 264:]
    h = torch.empty(37, 264, dtype=torch.bfloat16, device="cuda")
    swiglu.swiglu_rows(gate, up, h)
    assert torch.equal(h, swiglu.swiglu(gate.contiguous(), up.contiguous()))
    dh = torch.randn(37, 264, device="cuda", generator=g).to(torch.bfloat16)
    gbuf = torch.empty(37, 2 * 264, dtype=torch.bfloat16, device="cuda")
    swiglu.swiglu_bwd_rows(dh, gate, up, gbuf[:, :264], gbuf[:, 264:])
    dg, du = swiglu.SwiGLU.backward(
        type("C", (), {"saved_tensors": (gate.contiguous(), up.contiguous())})(), dh)
    assert torch.equal(gbuf[:, :264], dg) and torch.equal(gbuf[:, 264:], du)


def test_decoder_layer_takes_the_fused_path(monkeypatch):
    print("fused routing", flush=True)
    cfg, model = _model()
    hackathon_amd.apply()
    calls = {"qkv": 0, "mlp": 0}
    qkv_apply, mlp_apply = fused_proj.QKVRoPE.apply, fused_proj.LoraMLP.apply

    def count_qkv(*a):
        calls["qkv"] += 1
        return qkv_apply(*a)

    def count_mlp(*a):
        calls["mlp"] += 1
        return mlp_apply(*a)

    monkeypatch.setattr(fused_proj.QKVRoPE, "apply", count_qkv)
    monkeypatch.setattr(fused_proj.LoraMLP, "apply", count_mlp)
    ids = torch.randint(0, 1000, (2, 64), device="cuda")
    out = model(input_ids=ids, labels=ids, use_cache=False)
    out.loss.backward()
    assert calls == {"qkv": 1, "mlp": 1}
    assert all(p.grad is not None and torch.isfinite(p.grad).all()
               for p in qlora_step.lora_parameters(model))


def test_lora_pack_group_matches_the_single_packs():
    print("lora pack group", flush=True)
    from hackathon_amd import gemm

    g = torch.Generator(device="cuda").manual_seed(4)
    K, ns, scales = 256, (512, 128, 64), (2.0, 0.5, 1.5)
    facs = [(torch.randn(16, K, device="cuda", generator=g),
             torch.randn(n, 16, device="cuda", generator=g), s) for n, s in zip(ns, scales)]
    a16, at, bs, bt = gemm.lora_pack_group(facs, torch.bfloat16)
    assert torch.all(at[:, 48:] == 0)  # columns past the last slot
    off = 0
    for i, ((a, b, s), n) in enumerate(zip(facs, ns)):
        a1, at1, bs1, bt1 = gemm.lora_pack(a, b, s, torch.bfloat16, 64)
        cols = slice(16 * i, 16 * i + 16)
        assert torch.equal(a16[cols], a1)
        assert torch.equal(at[:, cols], at1[:, :16])
        rows = slice(off, off + n)
        assert torch.equal(bs[rows, cols], bs1[:, :16])
        others = torch.ones(64, dtype=torch.bool, device="cuda")
        others[cols] = False
        assert torch.all(bs[rows][:, others] == 0)
        assert torch.equal(bt[cols, rows], bt1)
        other_slots = torch.ones(48, dtype=torch.bool, device="cuda")
        other_slots[cols] = False
        assert torch.all(bt[other_slots][:, rows] == 0)  # block-diagonal
        off += n
    assert bt.shape == (48, sum(ns))
    assert torch.all(at[:, 48:] == 0)


@pytest.mark.parametrize("M,ns,scales", [
    (4096, (3584, 512, 512), (2.0, 2.0, 2.0)),   # Qwen2.5-7B q/k/v
    (300, (64, 128, 8, 40), (0.5, 1.0, 2.0, 3.0)),  # ragged tokens, four slots, unequal scalings
    (96, (256,), (1.5,)),
])
def test_lora_wgrad_diag_matches_per_adapter(M, ns, scales):
    """qlora_lora_wgrad_diag (one multi-slot pass over the concatenated output gradient) gives
    each adapter's lora_B gradient s_q g_q^T u_q: against the fp64 product within an fp32
    accumulation bound, as the per-adapter lora_wgrad is (the two sum in different orders)."""
    print(f"lora_wgrad_diag M={M} ns={ns}", flush=True)
    from hackathon_amd import gemm

    g = torch.Generator(device="cuda").manual_seed(7)
    G, N = len(ns), sum(ns)
    q = torch.randn(M, N, device="cuda", generator=g).to(torch.bfloat16)
    pt = gemm.lora_t_buffer(M, torch.bfloat16, "cuda", rows=16 * G)
    pt.copy_(torch.randn(16 * G, M, device="cuda", generator=g).to(torch.bfloat16))
    offs = [0]
    for n in ns:
        offs.append(offs[-1] + n)
    out = gemm.lora_wgrad_diag(pt, q, offs, scales)
    assert out.shape == (N, 16) and out.dtype == torch.float32
    for i, s in enumerate(scales):
        qi, pti = q[:, offs[i]:offs[i + 1]], pt[16 * i:16 * i + 16]
        ref = s * (qi.double().t() @ pti.double().t())
        got = out[offs[i]:offs[i + 1]].double()
        bound = 4e-6 * M ** 0.5 * s * (qi.double().t().abs() @ pti.double().t().abs()) + 1e-6
        assert torch.all((got - ref).abs() <= bound)
        # the per-adapter call sums in another order: both within the bound of the exact value
        sep = gemm.lora_wgrad(pti, qi, alpha=s).double()
        assert torch.all((sep - ref).abs() <= bound)
        assert torch.all((got - sep).abs() <= 2 * bound)


@pytest.mark.parametrize("rows,cols,dtype", [(4096, 18944, torch.bfloat16),
                                             (37, 1024, torch.bfloat16),
                                             (300, 96, torch.bfloat16),
                                             (1000, 2048, torch.float16)])
def test_swiglu_bwd_lora_down(rows, cols, dtype):
    """The fused SwiGLU backward writes the same gradient bits as qlora_swiglu_bwd_rows and the
    two scaled down-projections of them (fp32 accumulation bound vs fp64), zeros after column
    32, and the transposed copy exactly; ragged row counts exercise rows past M."""
    print(f"swiglu_bwd_lora_down {rows}x{cols} {dtype}", flush=True)
    from hackathon_amd import gemm

    g = torch.Generator(device="cuda").manual_seed(rows + cols)
    y = torch.randn(rows, 2 * cols, device="cuda", generator=g).to(dtype)
    gate, up = y[:, :cols], y[:, cols:]
    dh = torch.randn(rows, cols, device="cuda", generator=g).to(dtype)
    bt = (torch.randn(16, 2 * cols, device="cuda", generator=g) * 0.1).to(dtype)
    buf = torch.empty(rows, 2 * cols, dtype=dtype, device="cuda")
    du = torch.full((rows, 64), 5.0, dtype=dtype, device="cuda")
    dut = gemm.lora_t_buffer(rows, dtype, "cuda", rows=32)
    swiglu.swiglu_bwd_lora_down(dh, gate, up, buf[:, :cols], buf[:, cols:], bt[:, :cols],
                                bt[:, cols:], 2.0, 0.5, du, dut)
    ref = torch.empty_like(buf)
    swiglu.swiglu_bwd_rows(dh, gate, up, ref[:, :cols], ref[:, cols:])
    assert torch.equal(buf, ref)
    for q, (c0, a) in enumerate(((0, 2.0), (cols, 0.5))):
        x = ref[:, c0:c0 + cols].double()
        w = bt[:, c0:c0 + cols].double()
        exact = a * (x @ w.t())
        rnd = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11  # one rounding to the output
        bound = a * 4 * 2.0**-22 * cols * x.abs().max() * w.abs().max() + rnd * exact.abs()
        got = du[:, 16 * q:16 * q + 16].double()
        assert torch.all((got - exact).abs() <= bound), q
    assert torch.all(du[:, 32:] == 0)
    assert torch.equal(dut, du[:, :32].t())


@pytest.mark.parametrize("rows,cols,dtype", [(4096, 18944, torch.bfloat16),
                                             (37, 1024, torch.bfloat16),
                                             (300, 96, torch.bfloat16),
                                             (1000, 2048, torch.float16)])
def test_swiglu_fwd_lora_down(rows, cols, dtype):
    """qlora_swiglu_fwd_lora_down: h with the bits of qlora_swiglu_fwd_rows, u = alpha h a^T
    within the fp32 accumulation bound of an fp64 product, zeros after column 16, u_t the exact
    transpose; ragged row counts exercise rows past M."""
    print(f"swiglu_fwd_lora_down {rows}x{cols} {dtype}", flush=True)
    from hackathon_amd import gemm

    g = torch.Generator(device="cuda").manual_seed(5 * rows + cols)
    y = torch.randn(rows, 2 * cols, device="cuda", generator=g).to(dtype)
    gate, up = y[:, :cols], y[:, cols:]
    a = (torch.randn(16, cols, device="cuda", generator=g) * 0.05).to(dtype)
    h = torch.empty(rows, cols, dtype=dtype, device="cuda")
    u = torch.full((rows, 64), 5.0, dtype=dtype, device="cuda")
    ut = gemm.lora_t_buffer(rows, dtype, "cuda", rows=16)
    swiglu.swiglu_fwd_lora_down(gate, up, h, a, u, ut, alpha=0.75)
    ref = torch.empty_like(h)
    swiglu.swiglu_rows(gate, up, ref)
    assert torch.equal(h, ref)
    hd, ad = ref.double(), a.double()
    exact = 0.75 * (hd @ ad.t())
    rnd = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    bound = 0.75 * 4 * 2.0**-22 * cols * hd.abs().max() * ad.abs().max() + rnd * exact.abs()
    assert torch.all((u[:, :16].double() - exact).abs() <= bound)
    assert torch.all(u[:, 16:] == 0)
    assert torch.equal(ut, u[:, :16].t())


@pytest.mark.parametrize("rows,cols,dtype", [(4096, 18944, torch.bfloat16),
                                             (37, 1024, torch.bfloat16),
                                             (300, 96, torch.bfloat16),
                                             (1000, 2048, torch.float16),
                                             (4000, 4832, torch.bfloat16)])
def test_swiglu_bwd_lora(rows, cols, dtype):
    """qlora_swiglu_bwd_lora: the gradient bits of qlora_swiglu_bwd_rows, the two scaled
    down-projections of them (fp32 accumulation bound vs fp64, zeros after column 32, the
    transposed copy exactly) and both lora_B gradients beta d^T u^T (fp32 accumulation bound
    vs fp64). Row counts that are not a multiple of 32 leave rows of the last tile past M,
    which must not reach either product; 96 and 4832 columns leave a partial last block of
    256 columns."""
    print(f"swiglu_bwd_lora {rows}x{cols} {dtype}", flush=True)
    from hackathon_amd import gemm

    g = torch.Generator(device="cuda").manual_seed(3 * rows + cols)
    y = torch.randn(rows, 2 * cols, device="cuda", generator=g).to(dtype)
    gate, up = y[:, :cols], y[:, cols:]
    dh = torch.randn(rows, cols, device="cuda", generator=g).to(dtype)
    bt = (torch.randn(16, 2 * cols, device="cuda", generator=g) * 0.1).to(dtype)
    ut = gemm.lora_t_buffer(rows, dtype, "cuda", rows=32)
    ut.copy_(torch.randn(32, rows, device="cuda", generator=g).to(dtype))
    buf = torch.empty(rows, 2 * cols, dtype=dtype, device="cuda")
    du = torch.full((rows, 64), 5.0, dtype=dtype, device="cuda")
    dut = gemm.lora_t_buffer(rows, dtype, "cuda", rows=32)
    udt = gemm.lora_t_buffer(rows, dtype, "cuda", rows=16)
    udt.copy_(torch.randn(16, rows, device="cuda", generator=g).to(dtype))
    db_gate, db_up = swiglu.swiglu_bwd_lora(dh, gate, up, buf[:, :cols], buf[:, cols:],
                                            bt[:, :cols], bt[:, cols:], ut[:16], ut[16:32],
                                            2.0, 0.5, 2.0, 0.5, du, dut)
    ref = torch.empty_like(buf)
    swiglu.swiglu_bwd_rows(dh, gate, up, ref[:, :cols], ref[:, cols:])
    assert torch.equal(buf, ref)
    # with the down adapter's lora_A gradient: the same outputs, plus da = 1.5 ud^T h
    buf2 = torch.empty_like(buf)
    du2 = torch.full((rows, 64), 5.0, dtype=dtype, device="cuda")
    dut2 = gemm.lora_t_buffer(rows, dtype, "cuda", rows=32)
    db_gate2, db_up2, da = swiglu.swiglu_bwd_lora(
        dh, gate, up, buf2[:, :cols], buf2[:, cols:], bt[:, :cols], bt[:, cols:], ut[:16],
        ut[16:32], 2.0, 0.5, 2.0, 0.5, du2, dut2, ud_t=udt, beta_down=1.5)
    # (the dB partials come from fewer, longer row ranges here: fp32 rounding apart, checked
    # against fp64 with the others below)
    assert torch.equal(buf2, ref) and torch.equal(du2, du) and torch.equal(dut2, dut)
    h = torch.empty(rows, cols, dtype=dtype, device="cuda")
    swiglu.swiglu_rows(gate, up, h)
    hd, udd = h.double(), udt.double()
    exact_a = 1.5 * (udd @ hd)
    bound_a = 1.5 * 4 * 2.0**-22 * rows * hd.abs().max() * udd.abs().max()
    assert da.shape == (16, cols) and torch.all((da.double() - exact_a).abs() <= bound_a)
    u = ut.double()
    for q, (c0, a, db, db2) in enumerate(((0, 2.0, db_gate, db_gate2),
                                          (cols, 0.5, db_up, db_up2))):
        x = ref[:, c0:c0 + cols].double()
        w = bt[:, c0:c0 + cols].double()
        exact = a * (x @ w.t())
        rnd = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11  # one rounding to the output
        bound = a * 4 * 2.0**-22 * cols * x.abs().max() * w.abs().max() + rnd * exact.abs()
        got = du[:, 16 * q:16 * q + 16].double()
        assert torch.all((got - exact).abs() <= bound), q
        uq = u[16 * q:16 * q + 16]
        exact_b = a * (x.t() @ uq.t())
        bound_b = a * 4 * 2.0**-22 * rows * x.abs().max() * uq.abs().max()
        assert db.shape == (cols, 16) and db.dtype == torch.float32
        assert torch.all((db.double() - exact_b).abs() <= bound_b), q
        assert torch.all((db2.double() - exact_b).abs() <= bound_b), q
    assert torch.all(du[:, 32:] == 0)
    assert torch.equal(dut, du[:, :32].t())


@pytest.mark.parametrize("rows,cols,dtype", [(4096, 18944, torch.bfloat16),
                                             (37, 1024, torch.bfloat16),
                                             (1000, 2048, torch.float16),
                                             (300, 4832, torch.bfloat16)])
def test_swiglu_lora_dropout_kernels(rows, cols, dtype):
    """LoRA dropout of the down adapter inside the SwiGLU kernels: the forward stores h with the
    bits of qlora_swiglu_fwd_rows and keep bits equal to qlora_lora_dropout_scale_bits' on that
    h for the same seed (the oracle's Philox mask on small inputs), u = alpha xd a^T on the dropped
    h (within the fp32 bound of fp64); the backward gives the SwiGLU gradients, du and both dB of
    the dropout-free call bit for bit and da = beta ud^T xd from the same bits (fp32 bound)."""
    print(f"swiglu lora dropout {rows}x{cols} {dtype}", flush=True)
    import numpy as np

    from hackathon_amd import gemm
    from oracle import philox
    from _util import keep_rows

    p, seed = 0.05, 987654321
    g = torch.Generator(device="cuda").manual_seed(7 * rows + cols)
    y = torch.randn(rows, 2 * cols, device="cuda", generator=g).to(dtype)
    gate, up = y[:, :cols], y[:, cols:]
    a = (torch.randn(16, cols, device="cuda", generator=g) * 0.05).to(dtype)
    h = torch.empty(rows, cols, dtype=dtype, device="cuda")
    u = torch.full((rows, 64), 5.0, dtype=dtype, device="cuda")
    ut = gemm.lora_t_buffer(rows, dtype, "cuda", rows=16)
    bits = swiglu.swiglu_fwd_lora_down(gate, up, h, a, u, ut, alpha=0.75, p=p, seed=seed)
    ref_h = torch.empty_like(h)
    swiglu.swiglu_rows(gate, up, ref_h)
    assert torch.equal(h, ref_h)
    xd, ref_bits = lora.dropout_with_bits(ref_h, p, seed)
    assert np.array_equal(keep_rows(bits, rows), keep_rows(ref_bits, rows))
    if rows * cols <= 1 << 20:
        keep = philox.keep_mask(seed, rows, cols, p)
        assert np.array_equal(keep_rows(bits, rows), np.packbits(keep, axis=1, bitorder="little"))
    xdd, ad = xd.double(), a.double()
    exact = 0.75 * (xdd @ ad.t())
    rnd = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    bound = 0.75 * 4 * 2.0**-22 * cols * xdd.abs().max() * ad.abs().max() + rnd * exact.abs()
    assert torch.all((u[:, :16].double() - exact).abs() <= bound)
    assert torch.all(u[:, 16:] == 0) and torch.equal(ut, u[:, :16].t())

    dh = torch.randn(rows, cols, device="cuda", generator=g).to(dtype)
    bt = (torch.randn(16, 2 * cols, device="cuda", generator=g) * 0.1).to(dtype)
    utg = gemm.lora_t_buffer(rows, dtype, "cuda", rows=32)
    utg.copy_(torch.randn(32, rows, device="cuda", generator=g).to(dtype))
    udt = gemm.lora_t_buffer(rows, dtype, "cuda", rows=16)
    udt.copy_(torch.randn(16, rows, device="cuda", generator=g).to(dtype))
    outs = []
    for drop in (False, True):
        buf = torch.empty(rows, 2 * cols, dtype=dtype, device="cuda")
        du = torch.full((rows, 64), 5.0, dtype=dtype, device="cuda")
        dut = gemm.lora_t_buffer(rows, dtype, "cuda", rows=32)
        res = swiglu.swiglu_bwd_lora(dh, gate, up, buf[:, :cols], buf[:, cols:], bt[:, :cols],
                                     bt[:, cols:], utg[:16], utg[16:32], 2.0, 0.5, 2.0, 0.5, du,
                                     dut, ud_t=udt, beta_down=1.5,
                                     bits_down=bits if drop else None, p_down=p)
        outs.append((buf, du, dut) + tuple(res))
    (b0, du0, dut0, dbg0, dbu0, _), (b1, du1, dut1, dbg1, dbu1, da1) = outs
    assert torch.equal(b0, b1) and torch.equal(du0, du1) and torch.equal(dut0, dut1)
    assert torch.equal(dbg0, dbg1) and torch.equal(dbu0, dbu1)
    udd = udt.double()
    exact_a = 1.5 * (udd @ xdd)
    bound_a = 1.5 * 4 * 2.0**-22 * rows * xdd.abs().max() * udd.abs().max()
    assert da1.shape == (16, cols) and torch.all((da1.double() - exact_a).abs() <= bound_a)

    # the down adapter's input gradient through its mask, added on chip: every result equals the
    # separate masked add (lora.up_masked_add on a copy of dh) followed by the same call
    dud = (torch.randn(rows, 64, device="cuda", generator=g) * 0.5).to(dtype)
    dh_sum = dh.clone()
    lora.up_masked_add(dh_sum, dud, a, bits, p)
    dh_before = dh.clone()
    outs = []
    for fused in (False, True):
        buf = torch.empty(rows, 2 * cols, dtype=dtype, device="cuda")
        du = torch.full((rows, 64), 5.0, dtype=dtype, device="cuda")
        dut = gemm.lora_t_buffer(rows, dtype, "cuda", rows=32)
        res = swiglu.swiglu_bwd_lora(dh if fused else dh_sum, gate, up, buf[:, :cols],
                                     buf[:, cols:], bt[:, :cols], bt[:, cols:], utg[:16],
                                     utg[16:32], 2.0, 0.5, 2.0, 0.5, du, dut, ud_t=udt,
                                     beta_down=1.5, bits_down=bits, p_down=p,
                                     du_add=dud if fused else None, a_add=a if fused else None)
        outs.append((buf, du, dut) + tuple(res))
    for x0, x1 in zip(*outs):
        assert torch.equal(x0, x1)
    assert torch.equal(dh, dh_before)  # the sum is taken on chip, dh is not written
