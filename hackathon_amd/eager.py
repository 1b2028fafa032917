"""The unpatched PyTorch path of the 4-bit and LoRA layers, in plain torch ops.

This is what bitsandbytes' Linear4bit.forward and peft's 4-bit LoRA forward compute
(dequantise with torch ops, then F.linear in the compute dtype; base + B(A(dropout(x))) *
scaling). It serves two purposes only: the original path that a patched forward hands
unsupported inputs to (CPU or meta tensors, as solution/nf4.py:145-146 and
solution/lora.py:163-164 do), and the eager PyTorch-ROCm baseline of the QLoRA step that
the benchmark compares against. It never stands in for a HIP kernel on a GPU input the
kernels accept.
"""

from __future__ import annotations

import torch

from . import quant


def dequantize_eager(packed: torch.Tensor, state: quant.QuantState, dtype) -> torch.Tensor:
    """Torch-op NF4 dequantisation: nf4[code] * blockscale, rounded to `dtype`."""
    p = packed.reshape(-1)
    codes = torch.stack(((p >> 4) & 15, p & 15), dim=1).reshape(-1).long()
    n = codes.numel()
    scale = quant.absmax_of(state)
    w = quant.nf4_code(p.device)[codes].view(-1, state.blocksize) if n % state.blocksize == 0 \
        else None
    if w is not None:
        w = w * scale[:, None]
    else:
        w = quant.nf4_code(p.device)[codes] * scale.repeat_interleave(state.blocksize)[:n]
    return w.reshape(state.shape).to(dtype)


def linear4bit_eager(module, x):
    """bitsandbytes-style 4-bit forward: dequantise, F.linear in the compute dtype, cast back."""
    state = module.weight.quant_state
    inp_dtype = x.dtype
    cdt = module.compute_dtype or x.dtype
    w = dequantize_eager(module.weight.data, state, cdt)
    bias = module.bias.to(cdt) if module.bias is not None else None
    return torch.nn.functional.linear(x.to(cdt), w, bias).to(inp_dtype)


def lora_forward_eager(layer, x):
    """peft 4-bit LoRA forward: result = base(x) + lora_B(lora_A(dropout(x))) * scaling."""
    result = layer.base_layer(x)
    for a in layer.active_adapters:
        if layer.disable_adapters or layer.merged or a not in layer.lora_A:
            continue
        cdt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") \
            else (layer.compute_dtype or x.dtype)
        xd = layer.lora_dropout[a](x).to(cdt)
        lo = torch.nn.functional.linear(
            torch.nn.functional.linear(xd, layer.lora_A[a].weight.to(cdt)),
            layer.lora_B[a].weight.to(cdt))
        result = result + lo * layer.scaling[a]
    return result
