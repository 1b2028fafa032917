"""NF4 storage format: codebook, double-quant code map, QuantState, quantizer, 4-bit linear.

The reference takes all of this from bitsandbytes (`bnbf.get_4bit_type("nf4")`,
`QuantState`, `quantize_4bit`, `Linear4bit`; solution/nf4.py:58-60,65-68,73-86,118,156 and
solution/test_kernels.py:41-52), which is not available here. This module is the format
producer the dequant kernel consumes, with the attribute surface the façades read:

  packed   uint8 [n/2, 1]; byte i = (code of weight 2i) << 4 | (code of weight 2i+1)
  QuantState.absmax      uint8 [ceil(n/blocksize)]  codes of (absmax - offset)   (nested)
                         float32 [ceil(n/blocksize)] block absmax                 (plain)
  QuantState.offset      float32 0-d: the mean of the block absmax                (nested)
  QuantState.state2      QuantState(absmax=float32 [ceil(nblocks/256)], code=float32 [256],
                         blocksize=256)                                           (nested)

Codebook: NormalFloat-4 of the QLoRA paper (Dettmers et al. 2023, arXiv:2305.14314,
Section 3 and Appendix E): the 16 quantiles of N(0,1), 8 on the positive side and 7 on the
negative side plus an exact zero, scaled to [-1, 1]. The fp32 values below are the published
table; a test re-derives them from `scipy.stats.norm.ppf`.

Double-quant code map: the signed 8-bit dynamic map of "8-bit Optimizers via Block-wise
Quantization" (Dettmers et al. 2022): value = ±10^(e-6) * f for exponent e in 0..6 and
2^e linear fractions f at the midpoints of an even split of [0.1, 1], plus 0 and 1.

Quantisation rounds to the nearest code (ties to the lower code), normalising by the
reciprocal of the block absmax; GPU tensors go through the library's kernel, CPU tensors
through the same arithmetic in torch ops (identical bytes). Nothing of it is bit-compared with bitsandbytes (which is
not installed); dequantisation of whatever this produces is what must be bit-exact.
"""

from __future__ import annotations

import math

import torch

NF4_CODE = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)


def nf4_code(device=None) -> torch.Tensor:
    """The 16-entry NF4 codebook as float32 (index = 4-bit code)."""
    return torch.tensor(NF4_CODE, dtype=torch.float32, device=device)


def dynamic_map(signed: bool = True) -> torch.Tensor:
    """The 256-entry signed dynamic (tree) quantisation map used for the absmax codes."""
    values = [0.0, 1.0]
    n_exp = 7
    for e in range(n_exp):
        n_frac = 2 ** e if signed else 2 ** (e + 1)
        edges = torch.linspace(0.1, 1.0, n_frac + 1, dtype=torch.float64)
        mids = ((edges[:-1] + edges[1:]) / 2.0) * (10.0 ** (e - (n_exp - 1)))
        values += mids.tolist()
        if signed:
            values += (-mids).tolist()
    values += [0.0] * (256 - len(values))
    return torch.tensor(sorted(values), dtype=torch.float32)


def _nearest_code(x: torch.Tensor, code: torch.Tensor) -> torch.Tensor:
    """Index of the nearest entry of a sorted code (ties go to the lower code)."""
    mids = (code[:-1] + code[1:]) * 0.5
    return torch.bucketize(x, mids, right=False)


class QuantState:
    """The part of bitsandbytes' QuantState the NF4 path reads (solution/nf4.py:65-68,73-86)."""

    def __init__(self, absmax, shape=None, code=None, blocksize=64, quant_type="nf4",
                 dtype=torch.float32, offset=None, state2=None):
        self.absmax = absmax
        self.shape = torch.Size(shape) if shape is not None else None
        self.code = code
        self.blocksize = int(blocksize)
        self.quant_type = quant_type
        self.dtype = dtype
        self.offset = offset
        self.state2 = state2

    @property
    def nested(self) -> bool:
        return self.state2 is not None

    def to(self, device):
        self.absmax = self.absmax.to(device)
        if self.code is not None:
            self.code = self.code.to(device)
        if self.offset is not None:
            self.offset = self.offset.to(device)
        if self.state2 is not None:
            self.state2.to(device)
        return self


def quantize_blockwise_8bit(x: torch.Tensor, blocksize: int = 256):
    """8-bit blockwise quantisation with the dynamic map: returns (uint8 codes, QuantState)."""
    code = dynamic_map(True).to(x.device)
    flat = x.reshape(-1).float()
    n = flat.numel()
    nb = max(1, math.ceil(n / blocksize))
    padded = torch.zeros(nb * blocksize, dtype=torch.float32, device=x.device)
    padded[:n] = flat
    blocks = padded.view(nb, blocksize)
    absmax = blocks.abs().amax(dim=1)
    inv = torch.where(absmax > 0, 1.0 / absmax, torch.zeros_like(absmax))
    q = _nearest_code(blocks * inv[:, None], code).to(torch.uint8).reshape(-1)[:n]
    return q, QuantState(absmax=absmax, code=code, blocksize=blocksize, dtype=torch.float32)


def quantize_nf4(w: torch.Tensor, blocksize: int = 64, compress_statistics: bool = True,
                 blocksize2: int = 256):
    """NF4-quantise a weight tensor: returns (packed uint8 [n/2, 1], QuantState).

    GPU tensors are quantised by the library's kernel (qlora_nf4_quantize); CPU tensors by the
    same arithmetic in torch ops. Both give identical bytes: the double-quant offset, the mean
    of the block absmax, is accumulated in fp64 (exact for these values, so independent of
    the summation order) and rounded once to fp32."""
    if w.is_cuda and (not compress_statistics or blocksize2 == 256):
        return _quantize_nf4_gpu(w, blocksize, compress_statistics, blocksize2)
    flat = w.detach().reshape(-1).float()
    n = flat.numel()
    if n % 2:
        raise ValueError("NF4 packing needs an even number of weights")
    code = nf4_code(w.device)
    nb = math.ceil(n / blocksize)
    padded = torch.zeros(nb * blocksize, dtype=torch.float32, device=w.device)
    padded[:n] = flat
    blocks = padded.view(nb, blocksize)
    absmax = blocks.abs().amax(dim=1)
    inv = torch.where(absmax > 0, 1.0 / absmax, torch.zeros_like(absmax))
    idx = _nearest_code(blocks * inv[:, None], code).to(torch.uint8).reshape(-1)[:n]
    packed = ((idx[0::2] << 4) | idx[1::2]).reshape(-1, 1)
    if compress_statistics:
        offset = absmax.double().mean().float()
        qabs, state2 = quantize_blockwise_8bit(absmax - offset, blocksize2)
        state = QuantState(absmax=qabs, shape=w.shape, code=code, blocksize=blocksize,
                           dtype=w.dtype, offset=offset, state2=state2)
    else:
        state = QuantState(absmax=absmax, shape=w.shape, code=code, blocksize=blocksize,
                           dtype=w.dtype)
    return packed, state


def _quantize_nf4_gpu(w, blocksize, compress_statistics, blocksize2):
    from . import _lib

    x = w.detach()
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        x = x.float()
    x = x.contiguous()
    n = x.numel()
    if n % 2:
        raise ValueError("NF4 packing needs an even number of weights")
    dev = x.device
    nb = math.ceil(n / blocksize)
    code = nf4_code(dev)
    packed = torch.empty((n // 2, 1), dtype=torch.uint8, device=dev)
    nested = bool(compress_statistics)
    if nested:
        code2 = dynamic_map(True).to(dev)
        absmax = torch.empty(nb, dtype=torch.uint8, device=dev)
        absmax2 = torch.empty(math.ceil(nb / blocksize2), dtype=torch.float32, device=dev)
        offset = torch.empty((), dtype=torch.float32, device=dev)
    else:
        code2 = absmax2 = offset = None
        absmax = torch.empty(nb, dtype=torch.float32, device=dev)
    ws, ws_bytes = _lib.workspace("qlora_nf4_quantize_workspace_size", n, blocksize, int(nested),
                                  device=dev)
    _lib.call("qlora_nf4_quantize", x.data_ptr(), _lib.tag(x.dtype), n, blocksize, int(nested),
              blocksize2, code.data_ptr(), _lib.ptr(code2), packed.data_ptr(), absmax.data_ptr(),
              _lib.ptr(absmax2), _lib.ptr(offset), _lib.ptr(ws), ws_bytes, _lib.stream_of(x))
    if nested:
        state2 = QuantState(absmax=absmax2, code=code2, blocksize=blocksize2, dtype=torch.float32)
        state = QuantState(absmax=absmax, shape=w.shape, code=code, blocksize=blocksize,
                           dtype=w.dtype, offset=offset, state2=state2)
    else:
        state = QuantState(absmax=absmax, shape=w.shape, code=code, blocksize=blocksize,
                           dtype=w.dtype)
    return packed, state


def absmax_of(state: QuantState) -> torch.Tensor:
    """The fp32 block scales, reconstructed with the dequant kernel's operation order."""
    if not state.nested:
        return state.absmax.float()
    s2 = state.state2
    nb = state.absmax.numel()
    scale2 = s2.absmax.float().repeat_interleave(s2.blocksize)[:nb]
    return s2.code.float()[state.absmax.long()] * scale2 + state.offset.float()


class Params4bit(torch.nn.Parameter):
    """A frozen uint8 parameter holding packed NF4 codes, with its `quant_state`."""

    def __new__(cls, data, quant_state=None):
        self = torch.Tensor._make_subclass(cls, data, False)
        self.quant_state = quant_state
        return self

    def __deepcopy__(self, memo):
        return Params4bit(self.data.clone(), self.quant_state)


class Linear4bit(torch.nn.Module):
    """A linear layer with an NF4 weight, the attribute surface of bitsandbytes' Linear4bit
    that solution/nf4.py:115-149 reads: `weight` (packed, with `.quant_state`), `bias`,
    `compute_dtype`, `compute_type_is_set`, `set_compute_type`."""

    def __init__(self, in_features, out_features, bias=True, compute_dtype=None,
                 quant_type="nf4", device=None):
        super().__init__()
        if quant_type != "nf4":
            raise ValueError("only nf4 is implemented")
        self.in_features, self.out_features = in_features, out_features
        self.compute_dtype = compute_dtype
        self.compute_type_is_set = compute_dtype is not None
        self.quant_type = quant_type
        self.weight = None
        self.bias = (torch.nn.Parameter(torch.zeros(out_features, device=device),
                                        requires_grad=False) if bias else None)

    def set_compute_type(self, x):
        if self.compute_dtype is None:
            self.compute_dtype = x.dtype

    @classmethod
    def from_weight(cls, weight: torch.Tensor, bias=None, compute_dtype=None, blocksize=64,
                    compress_statistics=True):
        out_f, in_f = weight.shape
        layer = cls(in_f, out_f, bias=bias is not None, compute_dtype=compute_dtype,
                    device=weight.device)
        packed, state = quantize_nf4(weight, blocksize, compress_statistics)
        layer.weight = Params4bit(packed, state)
        if bias is not None:
            layer.bias = torch.nn.Parameter(bias.detach().clone(), requires_grad=False)
        return layer

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse)
        if self.weight is not None and getattr(self.weight, "quant_state", None) is not None:
            self.weight.quant_state.to(self.weight.device)  # the scales follow the codes
        return self

    def forward(self, x):
        from . import nf4

        return nf4.linear4bit(self, x)

    def extra_repr(self):
        return f"in_features={self.in_features}, out_features={self.out_features}, nf4"


LinearNF4 = Linear4bit
