"""MI355X (gfx950) QLoRA training-step kernel set with the reference's Python interface.

Drop-in for the reference's `solution` package (solution/__init__.py:1-34): the same module
names and function signatures, with every Triton kernel and every torch GEMM of the path
replaced by hand-written HIP kernels for gfx950 in `libqlora_gfx950.so` (C-ABI declared in
include/qlora_gfx950.h, bound through ctypes in `_lib`).

  nf4.py            NF4 dequant (+ double-quantised absmax) and the 4-bit linear
  rmsnorm.py        Qwen2RMSNorm.forward                      fwd + bwd
  rope.py           modeling_qwen2.apply_rotary_pos_emb        fwd + bwd (q and k in one launch)
  swiglu.py         Qwen2MLP.forward's silu(gate) * up         fwd + bwd
  lora.py           4-bit LoRA layer: dropout+cast, adapter GEMMs, scaled add
  fused_ce.py       chunked lm_head + CE with row selection (fused_head_loss)
  cross_entropy.py  chunked lm_head + CE installed on Qwen2ForCausalLM.forward
  quant.py          NF4 storage format: codebook, QuantState, quantizer, Linear4bit
  gemm.py           the MFMA GEMM behind every contraction of the path
  attention.py      causal flash attention behind transformers' "sdpa" entry (fwd + bwd)
  residual.py       Qwen2DecoderLayer with the residual adds fused into its two RMSNorms
  optim.py          FusedAdamW: AdamW over the adapters in one launch
  fused_proj.py     q/k/v (+ RoPE) and gate/up (+ SwiGLU) of a decoder layer as one LoRA GEMM each
  adapter_packs.py  every adapter group of a model packed in one launch per model forward
"""

PATCHES = ("rmsnorm", "rope", "cross_entropy", "lora", "attention", "residual")

_applied = set()


def apply(include_example=True):
    """Install every patch (idempotent), as solution/__init__.py:22-34 does; "attention",
    "residual" and "fused_proj" have no counterpart in the reference, which leaves attention to
    torch's SDPA, the decoder layer's residual adds to transformers and runs every projection
    as its own layer. "fused_proj" goes last: its forwards fall back to the ones installed
    before them. "adapter_packs" scopes each Qwen2Model forward so that the fused layers' adapter
    operands are packed in one launch."""
    from importlib import import_module

    for name in PATCHES:
        if name not in _applied:
            import_module(f"{__name__}.{name}").patch()
            _applied.add(name)
    if include_example and "swiglu" not in _applied:
        from .swiglu import patch_qwen2_mlp

        patch_qwen2_mlp()
        _applied.add("swiglu")
    if "fused_proj" not in _applied:
        from .fused_proj import patch as patch_fused_proj

        patch_fused_proj()
        _applied.add("fused_proj")
    if "adapter_packs" not in _applied:
        from .adapter_packs import patch as patch_adapter_packs

        patch_adapter_packs()
        _applied.add("adapter_packs")
