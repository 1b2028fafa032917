"""The SwiGLU kernels' sigmoid (hackathon_amd/csrc/ql_swiglu.h) divides with the hardware
reciprocal plus one Newton correction in fused multiply-adds wherever that equals the
correctly rounded fp32 division, and with the division elsewhere, so the kernels produce the
bits of 1 / (1 + exp(-x)) with a correctly rounded division (solution/swiglu.py:15-37 computes
tl.sigmoid in fp32). Exhaustive on the device through tests/support/recip_check.hip: every fp32
d in [1, 2^126) for the corrected reciprocal, and every one of the 2^32 fp32 bit patterns x for
the guarded sigmoid, scalar and eight-wide."""

import ctypes
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "support" / "_build" / "librecip_check.so"
ONE, TWO_126, INF = 0x3F800000, 0x7E800000, 0x7F800000


def _check(mode, lo, hi):
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built (python tests/support/build.py, or __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB))
    lib.recip_check.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64,
                                ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint32)]
    bad, first = ctypes.c_uint64(), ctypes.c_uint32()
    print(f"recip_check mode {mode} [{lo:#010x}, {hi:#011x})", flush=True)
    assert lib.recip_check(mode, lo, hi, ctypes.byref(bad), ctypes.byref(first)) == 0
    return bad.value, first.value


def test_corrected_reciprocal_is_the_correctly_rounded_division_below_2_126():
    bad, first = _check(0, ONE, TWO_126)
    assert bad == 0, f"{bad} mismatches, first {first:#010x}"


def test_corrected_reciprocal_differs_above_2_126_so_the_guard_is_needed():
    bad, first = _check(0, TWO_126, INF)
    assert bad > 0 and first >= TWO_126


def test_guarded_sigmoid_equals_the_division_for_every_fp32_input():
    bad, first = _check(1, 0, 1 << 32)
    assert bad == 0, f"{bad} mismatches, first x = {first:#010x}"
