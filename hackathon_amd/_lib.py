"""ctypes binding of libqlora_gfx950.so (the C-ABI declared in include/qlora_gfx950.h).

The library is loaded once, from this package directory only. There is no fallback: if the
library is missing, every kernel call raises, naming the build command. Each wrapper takes
torch tensors, checks what the C side cannot (device, dtype tags), and passes raw device
pointers plus the current HIP stream of the tensor's device.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libqlora_gfx950.so"

F32, F16, BF16 = 0, 1, 2
_DTYPE_TAG = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_ptr = ctypes.c_void_p
_c_f32 = ctypes.c_float
_c_u64 = ctypes.c_uint64
_c_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> argtypes; every function returns int (QL_OK = 0)
_SIGNATURES = {
    "qlora_nf4_dequant": [_c_ptr, _c_i64, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_f32, _c_int, _c_int,
                          _c_ptr, _c_ptr, _c_int, _c_ptr],
    "qlora_rmsnorm_fwd": [_c_ptr, _c_int, _c_i64, _c_ptr, _c_int, _c_ptr, _c_int, _c_i64, _c_ptr,
                          _c_i64, _c_i64, _c_f32, _c_ptr],
    "qlora_rmsnorm_bwd": [_c_ptr, _c_int, _c_i64, _c_ptr, _c_int, _c_i64, _c_ptr, _c_int, _c_ptr,
                          _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr],
    "qlora_rope_qk": [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int,
                      _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64p, _c_i64p, _c_i64p, _c_i64p,
                      _c_i64, _c_i64, _c_int, _c_ptr],
    "qlora_swiglu_fwd": [_c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_ptr],
    "qlora_swiglu_bwd": [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_ptr],
    "qlora_swiglu_fwd_rows": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64,
                              _c_int, _c_ptr],
    "qlora_swiglu_bwd_rows": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
                              _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr],
    "qlora_swiglu_bwd_lora_down": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
                                   _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_f32,
                                   _c_f32, _c_int, _c_ptr, _c_i64, _c_int, _c_ptr, _c_i64, _c_ptr,
                                   _c_i64, _c_ptr],
    "qlora_swiglu_bwd_lora": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
                              _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_ptr,
                              _c_ptr, _c_i64, _c_f32, _c_f32, _c_f32, _c_f32, _c_int, _c_ptr,
                              _c_i64, _c_int, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_f32,
                              _c_ptr, _c_ptr, _c_i64, _c_ptr],
    "qlora_swiglu_fwd_lora_down": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64,
                                   _c_i64, _c_ptr, _c_i64, _c_f32, _c_int, _c_ptr, _c_i64, _c_int,
                                   _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr],
    "qlora_swiglu_fwd_lora_down_dropout": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
                                           _c_i64, _c_i64, _c_ptr, _c_i64, _c_f32, _c_int,
                                           _c_ptr, _c_i64, _c_int, _c_ptr, _c_i64, _c_u64,
                                           _c_f32, _c_f32, _c_ptr, _c_i64, _c_ptr, _c_i64,
                                           _c_ptr],
    "qlora_swiglu_bwd_lora_dropout": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr,
                                      _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr,
                                      _c_i64, _c_ptr, _c_ptr, _c_i64, _c_f32, _c_f32, _c_f32,
                                      _c_f32, _c_int, _c_ptr, _c_i64, _c_int, _c_ptr, _c_i64,
                                      _c_ptr, _c_ptr, _c_ptr, _c_f32, _c_ptr, _c_ptr, _c_i64,
                                      _c_f32, _c_f32, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr,
                                      _c_i64, _c_ptr],
    "qlora_lora_dropout_scale": [_c_ptr, _c_int, _c_i64, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64,
                                 _c_u64, _c_f32, _c_f32, _c_ptr],
    "qlora_lora_scaled_add": [_c_ptr, _c_int, _c_i64, _c_ptr, _c_int, _c_i64, _c_ptr, _c_int,
                              _c_i64, _c_i64, _c_i64, _c_f32, _c_ptr],
    "qlora_lora_dropout_down": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                ctypes.POINTER(ctypes.c_uint64), _c_f32, _c_f32,
                                ctypes.POINTER(ctypes.c_void_p), _c_i64,
                                ctypes.POINTER(ctypes.c_void_p), _c_i64, _c_ptr, _c_i64, _c_int,
                                _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr],
    "qlora_lora_wgrad_masked": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                ctypes.POINTER(ctypes.c_void_p), _c_i64, _c_f32, _c_ptr, _c_f32,
                                _c_ptr, _c_i64, _c_ptr],
    "qlora_lora_dropout_scale_bits": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64,
                                      _c_i64, _c_int, _c_u64, _c_f32, _c_f32, _c_ptr],
    "qlora_lora_up_masked_add": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
                                 _c_i64, _c_i64, _c_int, _c_f32, _c_ptr],
    "qlora_lora_up_masked_add_slots": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
                                       ctypes.POINTER(ctypes.c_void_p), _c_i64, _c_int, _c_i64,
                                       _c_i64, _c_int, _c_f32, _c_ptr],
    "qlora_gemm": [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_int,
                   _c_ptr, _c_i64, _c_int, _c_ptr, _c_f32, _c_f32, _c_ptr],
    "qlora_gemm_ws": [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
                      _c_int, _c_ptr, _c_i64, _c_int, _c_ptr, _c_f32, _c_f32, _c_ptr, _c_i64,
                      _c_ptr],
    "qlora_nf4_dequant_t": [_c_ptr, _c_i64, _c_i64, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_f32, _c_int,
                            _c_int, _c_ptr, _c_ptr, _c_i64, _c_int, _c_ptr],
    "qlora_nf4_dequant_group": [_c_ptr, _c_int, _c_int, _c_ptr, _c_int, _c_ptr],
    "qlora_nf4_dequant_t_group": [_c_ptr, _c_int, _c_int, _c_ptr, _c_i64, _c_int, _c_ptr],
    "qlora_transpose16": [_c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr],
    "qlora_gemm_nt_cat": [_c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr,
                          _c_i64, _c_ptr, _c_i64, _c_int, _c_ptr, _c_i64, _c_int, _c_ptr, _c_f32,
                          _c_ptr, _c_i64, _c_ptr],
    "qlora_gemm_nt_cat_residual": [_c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
                                   _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_int, _c_ptr,
                                   _c_i64, _c_int, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr],
    "qlora_lora_down": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_ptr,
                        _c_i64, _c_int, _c_int, _c_f32, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr],
    "qlora_mfma_probe": [_c_ptr, _c_int, _c_int, _c_i64, _c_int, _c_ptr, _c_ptr, _c_ptr],
    "qlora_gemm_nf4": [_c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_int, _c_ptr,
                       _c_ptr, _c_f32, _c_int, _c_int, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr,
                       _c_i64, _c_int, _c_ptr, _c_i64, _c_ptr, _c_f32, _c_ptr, _c_i64, _c_ptr],
    "qlora_lora_wgrad_diag": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                              _c_i64p, ctypes.POINTER(ctypes.c_float), _c_ptr, _c_ptr, _c_i64,
                              _c_ptr],
    "qlora_lora_wgrad": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_ptr,
                         _c_int, _c_f32, _c_ptr, _c_i64, _c_ptr],
    "qlora_lora_wgrad_noalloc": [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                 _c_ptr, _c_int, _c_f32, _c_ptr],
    "qlora_lora_pack": [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_f32, _c_int, _c_ptr, _c_ptr, _c_ptr,
                        _c_ptr, _c_int, _c_ptr],
    "qlora_lora_pack_group": [_c_ptr, _c_int, _c_i64, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                              _c_int, _c_ptr],
    "qlora_lora_pack_jobs": [_c_ptr, _c_int, _c_i64, _c_ptr, _c_int, _c_int, _c_ptr],
    "qlora_nf4_quantize": [_c_ptr, _c_int, _c_i64, _c_int, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr,
                           _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_ptr],
    "qlora_add_rmsnorm_fwd": [_c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_ptr, _c_int, _c_ptr,
                              _c_i64, _c_ptr, _c_int, _c_i64, _c_ptr, _c_i64, _c_i64, _c_f32,
                              _c_ptr],
    "qlora_rmsnorm_bwd_residual": [_c_ptr, _c_int, _c_i64, _c_ptr, _c_int, _c_i64, _c_ptr, _c_int,
                                   _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr],
    "qlora_adamw_fp32": [_c_ptr, _c_int, _c_i64, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32,
                         _c_f32, _c_ptr],
    "qlora_attn_fwd": [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_i64,
                       _c_i64, _c_i64p, _c_i64p, _c_i64p, _c_i64p, _c_f32, _c_ptr],
    "qlora_attn_bwd": [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                       _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64p, _c_i64p, _c_i64p,
                       _c_i64p, _c_i64p, _c_i64p, _c_f32, _c_ptr, _c_i64, _c_ptr],
    "qlora_ce_rows": [_c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                      _c_ptr, _c_int, _c_int, _c_f32, _c_ptr],
    "qlora_ce_rows_scale_ptr": [_c_ptr, _c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr,
                                _c_ptr, _c_ptr, _c_int, _c_int, _c_ptr, _c_ptr],
}

# name -> argtypes; these return a byte count (int64)
_SIZE_QUERIES = {
    "qlora_gemm_workspace_size": [_c_int, _c_int, _c_i64, _c_i64, _c_i64],
    "qlora_gemm_nt_cat_workspace_size": [_c_i64, _c_i64, _c_i64],
    "qlora_gemm_nf4_workspace_size": [_c_i64, _c_i64, _c_i64],
    "qlora_lora_down_workspace_size": [_c_i64, _c_i64, _c_int],
    "qlora_lora_dropout_down_workspace_size": [_c_i64, _c_i64, _c_int],
    "qlora_lora_wgrad_workspace_size": [_c_i64, _c_i64, _c_int],
    "qlora_lora_wgrad_diag_workspace_size": [_c_i64, _c_i64, _c_int],
    "qlora_swiglu_bwd_lora_down_workspace_size": [_c_i64, _c_i64],
    "qlora_swiglu_bwd_lora_workspace_size": [_c_i64, _c_i64, _c_int],
    "qlora_swiglu_fwd_lora_down_workspace_size": [_c_i64, _c_i64],
    "qlora_nf4_quantize_workspace_size": [_c_i64, _c_int, _c_int],
    "qlora_attn_bwd_workspace_size": [_c_i64, _c_i64, _c_i64, _c_i64],
    "qlora_adamw_chunk_elems": [],
}

_lib = None
_lock = threading.Lock()


class KernelLibraryMissing(RuntimeError):
    pass


ABI_VERSION = 3  # qlora_abi_version() of the library these signatures describe


def load():
    """The loaded ctypes library (loads it on first use; raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise KernelLibraryMissing(
                f"{LIB_PATH.name} is not built: run `python -m hackathon_amd.build` "
                f"(expected at {LIB_PATH})")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        lib.qlora_strerror.argtypes = [ctypes.c_int]
        lib.qlora_strerror.restype = ctypes.c_char_p
        for name, argtypes in _SIZE_QUERIES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int64
        lib.qlora_abi_version.argtypes = []
        lib.qlora_abi_version.restype = ctypes.c_int
        lib.qlora_dropout_keep_threshold.argtypes = [ctypes.c_float]
        lib.qlora_dropout_keep_threshold.restype = ctypes.c_uint32
        version = lib.qlora_abi_version()
        if version != ABI_VERSION:
            raise KernelLibraryMissing(
                f"{LIB_PATH.name} has C-ABI version {version}, these bindings expect "
                f"{ABI_VERSION}: rebuild it with `python -m hackathon_amd.build`")
        _lib = lib
    return _lib


def exported_symbols():
    """Names the binding expects the library to export (used by the ABI tests)."""
    return sorted(list(_SIGNATURES) + list(_SIZE_QUERIES) + [
        "qlora_strerror", "qlora_abi_version", "qlora_dropout_keep_threshold"])


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().qlora_strerror(status).decode()
        raise RuntimeError(f"{what} failed with status {status}: {msg}")


def tag(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_TAG[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}") from None


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("HIP kernels need tensors on a GPU device")


def require_rows(dtype: torch.dtype, **tensors: torch.Tensor | None) -> None:
    """Each named tensor (None skips it) is a 2-D matrix on a GPU, of `dtype`, with unit stride
    along its rows: what the C-ABI's single dtype tag and row-stride arguments describe. Raises
    TypeError (dtype) or ValueError (device, layout) naming the tensor."""
    for name, t in tensors.items():
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a GPU device")
        if t.dtype != dtype:
            raise TypeError(f"{name} is {t.dtype}; this call takes {dtype} operands")
        if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
            raise ValueError(f"{name} must be a 2-D matrix with unit stride along its rows")


def i64_array(values) -> ctypes.Array:
    return (ctypes.c_int64 * len(values))(*[int(v) for v in values])


class LoraFactor(ctypes.Structure):
    """ql_lora_factor: one adapter's fp32 factors A [16, K], B [n, 16] and its scaling."""
    _fields_ = [("A", ctypes.c_void_p), ("B", ctypes.c_void_p), ("n", ctypes.c_int64),
                ("scaling", ctypes.c_float)]


def lora_factors(items) -> ctypes.Array:
    """A host array of ql_lora_factor from (A tensor, B tensor, scaling) triples."""
    arr = (LoraFactor * len(items))()
    for i, (a, b, s) in enumerate(items):
        arr[i] = LoraFactor(a.data_ptr(), b.data_ptr(), b.shape[0], float(s))
    return arr


class LoraPackJob(ctypes.Structure):
    """ql_lora_pack_job: one group of qlora_lora_pack_jobs (outputs as byte offsets)."""
    _fields_ = [("A", ctypes.c_void_p * 4), ("B", ctypes.c_void_p * 4), ("n", ctypes.c_int64 * 4),
                ("scaling", ctypes.c_float * 4), ("K", ctypes.c_int64), ("a16", ctypes.c_int64),
                ("at_pad", ctypes.c_int64), ("bs_pad", ctypes.c_int64), ("bt", ctypes.c_int64),
                ("count", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class Nf4Weight(ctypes.Structure):
    """ql_nf4_weight: one NF4 weight [rows, cols], its scales and its output."""
    _fields_ = [("packed", ctypes.c_void_p), ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
                ("absmax", ctypes.c_void_p), ("code2", ctypes.c_void_p),
                ("absmax2", ctypes.c_void_p), ("offset", ctypes.c_float),
                ("blocksize", ctypes.c_int), ("blocksize2", ctypes.c_int),
                ("out", ctypes.c_void_p)]


def workspace(name: str, *sizes, device) -> tuple:
    """(fp32 tensor or None, bytes) holding the workspace the size query `name` asks for,
    from torch's caching allocator (16-B aligned)."""
    nbytes = int(getattr(load(), name)(*sizes))
    if nbytes <= 0:
        return None, 0
    return torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=device), nbytes


def call(name: str, *args) -> None:
    """Call a C-ABI entry point and raise RuntimeError on a non-zero status."""
    check(getattr(load(), name)(*args), name)
