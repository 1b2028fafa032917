// Shared device helpers for the gfx950 QLoRA kernel library (libqlora_gfx950.so).
//
// Every kernel in this library is written for CDNA4 (gfx950): 64-lane wavefronts,
// 16-byte global accesses, LDS for tables and tiles, bf16 MFMA for contractions.
// Storage types are plain bits (uint16_t for bf16 and fp16) so that every conversion
// is explicit and its rounding is known.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qlora_gfx950.h"

#define QL_DEV __device__ __forceinline__

// ---------------------------------------------------------------------------------------
// Scalar conversions. f32 -> bf16 and f32 -> f16 are round-to-nearest-even, the rounding
// torch's `.to(torch.bfloat16)` / `.to(torch.float16)` performs; gfx950 lowers them to
// v_cvt_pk_bf16_f32 / v_cvt_f16_f32.
// ---------------------------------------------------------------------------------------
QL_DEV float bf16_bits_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

QL_DEV uint16_t f32_to_bf16_bits(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}

QL_DEV float f16_bits_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

QL_DEV uint16_t f32_to_f16_bits(float f) {
  // The value is an fp32 result when it is converted: without the empty register barrier the
  // AMDGPU backend may fuse the multiply that produced it with this conversion into one
  // v_fma_mixlo_f16 (a single rounding), and does so at some call sites and not at others,
  // so two kernels that evaluate the same expression would disagree in the last fp16 bit.
  asm("" : "+v"(f));
  _Float16 h = (_Float16)f;
  return __builtin_bit_cast(uint16_t, h);
}

// Two fp32 -> one packed 32-bit word of bf16 (lo in bits 0..15), RNE.
// One v_cvt_pk_bf16_f32 converts both values (the same RNE rounding as f32_to_bf16_bits; the
// scalar form costs a conversion per value plus the shift and or that join them).
QL_DEV uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

QL_DEV uint32_t pack_f16x2(float lo, float hi) {
  return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
}

// ---------------------------------------------------------------------------------------
// Element access by runtime dtype tag, resolved at compile time through templates.
// DT is one of QL_F32 / QL_F16 / QL_BF16 from the public header.
// ---------------------------------------------------------------------------------------
template <int DT> struct Elem;
template <> struct Elem<QL_F32> {
  using T = float;
  static QL_DEV float load(const T* p, int64_t i) { return p[i]; }
  static QL_DEV void store(T* p, int64_t i, float v) { p[i] = v; }
  static QL_DEV float to_f32(T v) { return v; }
  static QL_DEV T from_f32(float v) { return v; }
};
template <> struct Elem<QL_F16> {
  using T = uint16_t;
  static QL_DEV float load(const T* p, int64_t i) { return f16_bits_to_f32(p[i]); }
  static QL_DEV void store(T* p, int64_t i, float v) { p[i] = f32_to_f16_bits(v); }
  static QL_DEV float to_f32(T v) { return f16_bits_to_f32(v); }
  static QL_DEV T from_f32(float v) { return f32_to_f16_bits(v); }
};
template <> struct Elem<QL_BF16> {
  using T = uint16_t;
  static QL_DEV float load(const T* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  static QL_DEV void store(T* p, int64_t i, float v) { p[i] = f32_to_bf16_bits(v); }
  static QL_DEV float to_f32(T v) { return bf16_bits_to_f32(v); }
  static QL_DEV T from_f32(float v) { return f32_to_bf16_bits(v); }
};

// Round an fp32 value through a 16-bit type and back (RMSNorm's `.to(input_dtype)`).
template <int DT> QL_DEV float round_through(float v) {
  if constexpr (DT == QL_F32) return v;
  else return Elem<DT>::to_f32(Elem<DT>::from_f32(v));
}

// ---------------------------------------------------------------------------------------
// Wavefront reductions (64 lanes) with DPP/permute shuffles.
// ---------------------------------------------------------------------------------------
QL_DEV float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

QL_DEV float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Host-side helpers used by every entry point.
static inline int ql_hip_status(hipError_t e) { return e == hipSuccess ? QL_OK : (int)e; }

static inline bool ql_aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Whether the byte ranges spanned by two row-strided matrices of `rows` x `cols` elements of
// `elem` bytes (leading dimensions lda, ldb) intersect. Conservative for interleaved strided
// matrices: it compares the spans, not the elements.
static inline bool ql_spans_overlap(const void* a, int64_t lda, const void* b, int64_t ldb,
                                    int64_t rows, int64_t cols, int64_t elem) {
  if (rows <= 0 || cols <= 0) return false;
  const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
  const uintptr_t a1 = a0 + (uintptr_t)(((rows - 1) * lda + cols) * elem);
  const uintptr_t b1 = b0 + (uintptr_t)(((rows - 1) * ldb + cols) * elem);
  return a0 < b1 && b0 < a1;
}

static inline int ql_launch_status() { return ql_hip_status(hipGetLastError()); }

#define QL_DISPATCH_DTYPE(dt, DTC, ...)                  \
  switch (dt) {                                          \
    case QL_F32: { constexpr int DTC = QL_F32; __VA_ARGS__; break; } \
    case QL_F16: { constexpr int DTC = QL_F16; __VA_ARGS__; break; } \
    case QL_BF16: { constexpr int DTC = QL_BF16; __VA_ARGS__; break; } \
    default: return QL_EDTYPE;                           \
  }
