// LoRA elementwise kernels around the adapter GEMMs, for gfx950.
//
// Reference semantics:
//   solution/lora.py:29-46  OUT = IN * keep * scale (keep from a counter-based RNG), or a
//                           plain scale-and-cast when dropout is off;
//   solution/lora.py:49-60  OUT = BASE + LO * scaling in fp32.
//
// The dropout mask is regenerated (never stored): keep = U(seed, row*N + col) > p, with U the
// Philox4x32-10 uniform Triton's tl.rand(seed, int32 offset) draws (ql_philox.h), so a seed
// gives the reference's mask. The kernels test the equivalent integer condition on the folded
// Philox word against a threshold the host derives from p.
//
// HBM-bound. One workgroup per row; each thread moves 8 consecutive elements per step.
#include "ql_philox.h"
#include "ql_vec.h"

namespace {

constexpr int kThreads = 256;

using ql_philox::keep_word;
using ql_philox::philox_word0;

template <int IT, int OT, bool DROPOUT, bool VEC>
__global__ __launch_bounds__(kThreads) void dropout_scale_kernel(
    const typename Elem<IT>::T* __restrict__ in, int64_t in_rs, typename Elem<OT>::T* __restrict__ out,
    int64_t out_rs, int64_t n_cols, uint64_t seed, uint32_t thr, float scale) {
  const int64_t row = blockIdx.x;
  const auto* src = in + row * in_rs;
  auto* dst = out + row * out_rs;
  if constexpr (VEC) {
    for (int64_t c = 8 * (int64_t)threadIdx.x; c < n_cols; c += 8 * kThreads) {
      float v[8];
      Vec8<IT>::load(src + c, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (DROPOUT) {
          const uint32_t flat = (uint32_t)(row * n_cols + c + j);
          const bool keep = keep_word(philox_word0(flat, seed), thr);
          v[j] = keep ? v[j] * scale : 0.0f;
        } else {
          v[j] = v[j] * scale;
        }
      }
      Vec8<OT>::store(dst + c, v);
    }
  } else {
    for (int64_t c = threadIdx.x; c < n_cols; c += kThreads) {
      float v = Elem<IT>::to_f32(src[c]);
      if constexpr (DROPOUT) {
        const uint32_t flat = (uint32_t)(row * n_cols + c);
        v = keep_word(philox_word0(flat, seed), thr) ? v * scale : 0.0f;
      } else {
        v = v * scale;
      }
      dst[c] = Elem<OT>::from_f32(v);
    }
  }
}

// The dropout forward for the fused 4-bit LoRA layer: the same OUT = IN * keep * scale as
// dropout_scale_kernel (vector rows only), plus the keep mask as bits in the 8 x 8 block layout
// of ql_philox.h (bit j of a row's byte for columns c .. c + 7 is column c + j), so the backward
// needs no second Philox pass.
template <int IT, int OT>
__global__ __launch_bounds__(kThreads) void dropout_bits_kernel(
    const typename Elem<IT>::T* __restrict__ in, int64_t in_rs, typename Elem<OT>::T* __restrict__ out,
    int64_t out_rs, uint8_t* __restrict__ bits, int64_t bits_gs, int64_t n_cols, uint64_t seed,
    uint32_t thr, float scale) {
  const int64_t row = blockIdx.x;
  const auto* src = in + row * in_rs;
  auto* dst = out + row * out_rs;
  for (int64_t c = 8 * (int64_t)threadIdx.x; c < n_cols; c += 8 * kThreads) {
    float v[8];
    Vec8<IT>::load(src + c, v);
    uint32_t b = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t flat = (uint32_t)(row * n_cols + c + j);
      const bool keep = keep_word(philox_word0(flat, seed), thr);
      v[j] = keep ? v[j] * scale : 0.0f;
      b |= (uint32_t)keep << j;
    }
    Vec8<OT>::store(dst + c, v);
    bits[ql_philox::keep_byte(row, c, bits_gs)] = (uint8_t)b;
  }
}

// The dropout backward of G adapters' input gradients (the adapters of a group that read the
// same input, each with its own mask), added to the base gradient in one pass:
//   dx[m, k] += scale * sum_{g < G, keep_g(m, k)} sum_{r < 16} du[m, 16 g + r] * A[16 g + r, k]
// (du = s g B [M, >= 16 G], A [16 G, K] in dx's dtype; keep_g from adapter g's forward bits).
// A wave owns 64 columns and walks `row_blocks` blocks of 16 rows:
//  - products: each rank-16 sum is one v_mfma_f32_16x16x16 per 16 x 16 block and adapter
//    (exact 16-bit products summed in fp32), computed transposed, (du A)^T = A^T du^T, so a
//    lane's four results are four consecutive columns of one row; they go to the wave's LDS
//    area as one 16-B store, one adapter at a time (A's fragments for the 64 columns stay in
//    registers);
//  - the add: lane l takes 8 consecutive columns of row l / 8 (and l / 8 + 8), so every dx
//    access is 16 B and 8 lanes cover a 128-B row piece: the kept adapters' products are added
//    in fp32 in slot order from -0.0 (the additive identity of every float: an element no
//    adapter keeps gets dx + scale * -0.0 = dx exactly) and dx is rounded once.
// dx and the masks of the next row block are loaded while this one is computed. Measured on
// MI355X at 4096 x 3584: three adapters with 8 v_dot2_f32_bf16 per element and adapter took
// 34.5 us (the dot products are the bound); products straight from the MFMA registers to dx,
// as 8-B pieces of 16 rows per instruction, 53 us; all adapters' products in LDS at once (52 KB
// a workgroup at G = 3) 32 us.

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

template <int DT> QL_DEV f32x4_t mfma16(const uint2& a, const uint2& b);
template <> QL_DEV f32x4_t mfma16<QL_BF16>(const uint2& a, const uint2& b) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(v4i16_t, a),
                                                  __builtin_bit_cast(v4i16_t, b),
                                                  f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
}
template <> QL_DEV f32x4_t mfma16<QL_F16>(const uint2& a, const uint2& b) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                              __builtin_bit_cast(f16x4_t, b),
                                              f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
}

struct SlotBits {
  const uint8_t* p[4];  // adapter g's keep bits (8 x 8 blocks, ql_philox.h), one group stride
};

constexpr int kMaskedCols = 64;      // columns per wave (four 16-column blocks)
constexpr int kMaskedPitch = 64 + 4;  // floats per LDS row (padding spreads the 16-B stores)

// Each wave stages its products in its own LDS area, and the LDS accesses of one wave execute
// in program order, so the exchange between its lanes needs no workgroup barrier, only that the
// compiler keeps the reads after the writes (and the next writes after the reads).
QL_DEV void wave_lds_order() { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); }

template <int DT, int G>
__device__ __forceinline__ void up_masked_add_body(
    uint16_t* __restrict__ dx, int64_t dx_rs, const uint16_t* __restrict__ du, int64_t du_rs,
    const uint16_t* __restrict__ A, int64_t a_rs, const SlotBits& bits, int64_t bits_gs,
    int64_t M, int64_t K, float scale, int row_blocks,
    float (*__restrict__ prod)[16 * kMaskedPitch]) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int fr = lane & 15, fq = lane >> 4;
  const int64_t k0 = ((int64_t)blockIdx.x * (kThreads / 64) + wave) * kMaskedCols;
  const bool wave_on = k0 < K;  // wave-uniform
  // A^T fragments of block t, adapter g: A[16 g + 4 fq + i][k0 + 16 t + fr], i = 0 .. 3 (zero
  // past K: those products are never added)
  uint2 af[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int64_t k = k0 + 16 * t + fr;
      uint16_t h[4] = {0, 0, 0, 0};
      if (wave_on && k < K) {
#pragma unroll
        for (int i = 0; i < 4; ++i) h[i] = A[(16 * g + 4 * fq + i) * a_rs + k];
      }
      af[g][t] = make_uint2(h[0] | (uint32_t)h[1] << 16, h[2] | (uint32_t)h[3] << 16);
    }
  const int64_t mb0 = (int64_t)blockIdx.y * row_blocks * 16;
  int nb = row_blocks;
  if (mb0 + 16 * (int64_t)nb > M) nb = (int)((M - mb0 + 15) / 16);
  // the add's share of a block: rows hr and hr + 8, columns k0 + c8 .. +7
  const int hr = lane >> 3, c8 = (lane & 7) * 8;
  const bool col_ok = wave_on && k0 + c8 < K;  // K % 8 == 0: all 8 columns or none
  auto load_add = [&](int64_t mb, uint4* xv, uint32_t* bv) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t m = mb + hr + 8 * h < M ? mb + hr + 8 * h : M - 1;
      xv[h] = col_ok ? *reinterpret_cast<const uint4*>(dx + m * dx_rs + k0 + c8)
                     : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int g = 0; g < G; ++g)
        bv[2 * g + h] = col_ok ? bits.p[g][ql_philox::keep_byte(m, k0 + c8, bits_gs)] : 0u;
    }
  };
  uint4 xv[2];
  uint32_t bv[2 * G];
  load_add(mb0, xv, bv);
  for (int rb = 0; rb < nb; ++rb) {
    const int64_t mb = mb0 + 16 * rb;
    uint4 xn[2];
    uint32_t bn[2 * G];
    load_add(rb + 1 < nb ? mb + 16 : mb, xn, bn);
    const int64_t mp = mb + fr < M ? mb + fr : M - 1;  // the products' row (clamped)
    float sum[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 8; ++j) sum[h][j] = -0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      // adapter g's products of this block into the wave's LDS area: row fr, columns
      // 16 t + 4 fq .. +3
      const uint2 dv = wave_on ? *reinterpret_cast<const uint2*>(du + mp * du_rs + 16 * g + 4 * fq)
                               : make_uint2(0, 0);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f32x4_t p = mfma16<DT>(af[g][t], dv);
        *reinterpret_cast<f32x4_t*>(&prod[wave][fr * kMaskedPitch + 16 * t + 4 * fq]) = p;
      }
      wave_lds_order();  // the products are in this wave's LDS area
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float* pr = &prod[wave][(hr + 8 * h) * kMaskedPitch + c8];
        const f32x4_t p0 = *reinterpret_cast<const f32x4_t*>(pr);
        const f32x4_t p1 = *reinterpret_cast<const f32x4_t*>(pr + 4);
        const float pv[8] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
        const uint32_t b = bv[2 * g + h];
#pragma unroll
        for (int j = 0; j < 8; ++j) sum[h][j] = sum[h][j] + ((b >> j) & 1u ? pv[j] : -0.0f);
      }
      wave_lds_order();  // every read of these products is done before the next writes
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float v[8];
      Vec8<DT>::unpack(xv[h], v);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = v[j] + scale * sum[h][j];
      if (col_ok && mb + hr + 8 * h < M)
        *reinterpret_cast<uint4*>(dx + (mb + hr + 8 * h) * dx_rs + k0 + c8) = Vec8<DT>::pack(v);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) xv[h] = xn[h];
#pragma unroll
    for (int i = 0; i < 2 * G; ++i) bv[i] = bn[i];
  }
}

// One to three adapters (the groups of a Qwen2 layer) fit 128 registers: four waves a SIMD, so
// the 4096 x 3584 grid runs in one round. Four adapters need more and get their own kernel.
template <int DT, int G>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 8)))
void up_masked_add_kernel(uint16_t* __restrict__ dx, int64_t dx_rs,
                          const uint16_t* __restrict__ du, int64_t du_rs,
                          const uint16_t* __restrict__ A, int64_t a_rs, SlotBits bits,
                          int64_t bits_gs, int64_t M, int64_t K, float scale, int row_blocks) {
  __shared__ __attribute__((aligned(16))) float prod[kThreads / 64][16 * kMaskedPitch];
  up_masked_add_body<DT, G>(dx, dx_rs, du, du_rs, A, a_rs, bits, bits_gs, M, K, scale,
                            row_blocks, prod);
}

template <int DT>
__global__ __launch_bounds__(kThreads)
void up_masked_add4_kernel(uint16_t* __restrict__ dx, int64_t dx_rs,
                           const uint16_t* __restrict__ du, int64_t du_rs,
                           const uint16_t* __restrict__ A, int64_t a_rs, SlotBits bits,
                           int64_t bits_gs, int64_t M, int64_t K, float scale, int row_blocks) {
  __shared__ __attribute__((aligned(16))) float prod[kThreads / 64][16 * kMaskedPitch];
  up_masked_add_body<DT, 4>(dx, dx_rs, du, du_rs, A, a_rs, bits, bits_gs, M, K, scale,
                            row_blocks, prod);
}

template <int BT, int LT, int OT, bool VEC>
__global__ __launch_bounds__(kThreads) void scaled_add_kernel(
    const typename Elem<BT>::T* __restrict__ base, int64_t b_rs, const typename Elem<LT>::T* __restrict__ lo,
    int64_t l_rs, typename Elem<OT>::T* __restrict__ out, int64_t o_rs, int64_t n_cols, float scaling) {
  const int64_t row = blockIdx.x;
  const auto* b = base + row * b_rs;
  const auto* l = lo + row * l_rs;
  auto* o = out + row * o_rs;
  if constexpr (VEC) {
    for (int64_t c = 8 * (int64_t)threadIdx.x; c < n_cols; c += 8 * kThreads) {
      float bv[8], lv[8], ov[8];
      Vec8<BT>::load(b + c, bv);
      Vec8<LT>::load(l + c, lv);
#pragma unroll
      for (int j = 0; j < 8; ++j) ov[j] = bv[j] + lv[j] * scaling;
      Vec8<OT>::store(o + c, ov);
    }
  } else {
    for (int64_t c = threadIdx.x; c < n_cols; c += kThreads)
      o[c] = Elem<OT>::from_f32(Elem<BT>::to_f32(b[c]) + Elem<LT>::to_f32(l[c]) * scaling);
  }
}

bool rows_vec_ok(const void* p, int64_t rs, int dt, int64_t n_cols) {
  return (n_cols % 8) == 0 && ql_aligned(p, 16) && ((rs * ql_elem_size(dt)) % 16) == 0;
}

template <int IT, int OT>
int launch_dropout(const void* in, int64_t in_rs, void* out, int64_t out_rs, int64_t n_rows,
                   int64_t n_cols, uint64_t seed, float p, float scale, bool vec, hipStream_t s) {
  using I = typename Elem<IT>::T;
  using O = typename Elem<OT>::T;
  const dim3 grid((unsigned)n_rows);
  const bool drop = p > 0.0f;
#define QL_DROP(D, V)                                                                        \
  hipLaunchKernelGGL((dropout_scale_kernel<IT, OT, D, V>), grid, dim3(kThreads), 0, s,       \
                     (const I*)in, in_rs, (O*)out, out_rs, n_cols, seed, thr, scale)
  const uint32_t thr = drop ? ql_philox::keep_threshold(p) : 0u;
  if (drop) {
    if (vec) QL_DROP(true, true); else QL_DROP(true, false);
  } else {
    if (vec) QL_DROP(false, true); else QL_DROP(false, false);
  }
#undef QL_DROP
  return ql_launch_status();
}

template <int BT, int LT>
int launch_add(const void* base, int64_t b_rs, const void* lo, int64_t l_rs, void* out,
               int64_t o_rs, int64_t n_rows, int64_t n_cols, float scaling, bool vec,
               hipStream_t s) {
  constexpr int OT = (BT == LT) ? BT : QL_F32;
  using Bt = typename Elem<BT>::T;
  using Lt = typename Elem<LT>::T;
  using Ot = typename Elem<OT>::T;
  const dim3 grid((unsigned)n_rows);
  if (vec)
    hipLaunchKernelGGL((scaled_add_kernel<BT, LT, OT, true>), grid, dim3(kThreads), 0, s,
                       (const Bt*)base, b_rs, (const Lt*)lo, l_rs, (Ot*)out, o_rs, n_cols, scaling);
  else
    hipLaunchKernelGGL((scaled_add_kernel<BT, LT, OT, false>), grid, dim3(kThreads), 0, s,
                       (const Bt*)base, b_rs, (const Lt*)lo, l_rs, (Ot*)out, o_rs, n_cols, scaling);
  return ql_launch_status();
}

}  // namespace

extern "C" int qlora_lora_dropout_scale(const void* in, int in_dtype, int64_t in_row_stride,
                                        void* out, int out_dtype, int64_t out_row_stride,
                                        int64_t n_rows, int64_t n_cols, uint64_t seed, float p,
                                        float scale, ql_stream_t stream) {
  if (n_rows < 0 || n_cols < 0 || n_rows > UINT32_MAX) return QL_EINVAL;
  if (!ql_valid_dtype(in_dtype) || !ql_valid_dtype(out_dtype)) return QL_EDTYPE;
  if (n_rows == 0 || n_cols == 0) return QL_OK;
  if (!in || !out) return QL_EINVAL;
  const bool vec = rows_vec_ok(in, in_row_stride, in_dtype, n_cols) &&
                   rows_vec_ok(out, out_row_stride, out_dtype, n_cols);
  QL_DISPATCH_DTYPE2(in_dtype, out_dtype, IT, OT,
                     return launch_dropout<IT, OT>(in, in_row_stride, out, out_row_stride, n_rows,
                                                   n_cols, seed, p, scale, vec,
                                                   static_cast<hipStream_t>(stream)));
  return QL_EDTYPE;
}

extern "C" int qlora_lora_scaled_add(const void* base, int base_dtype, int64_t base_row_stride,
                                     const void* lo, int lo_dtype, int64_t lo_row_stride,
                                     void* out, int out_dtype, int64_t out_row_stride,
                                     int64_t n_rows, int64_t n_cols, float scaling,
                                     ql_stream_t stream) {
  if (n_rows < 0 || n_cols < 0 || n_rows > UINT32_MAX) return QL_EINVAL;
  if (!ql_valid_dtype(base_dtype) || !ql_valid_dtype(lo_dtype) ||
      out_dtype != ql_promote(base_dtype, lo_dtype))
    return QL_EDTYPE;
  if (n_rows == 0 || n_cols == 0) return QL_OK;
  if (!base || !lo || !out) return QL_EINVAL;
  const bool vec = rows_vec_ok(base, base_row_stride, base_dtype, n_cols) &&
                   rows_vec_ok(lo, lo_row_stride, lo_dtype, n_cols) &&
                   rows_vec_ok(out, out_row_stride, out_dtype, n_cols);
  QL_DISPATCH_DTYPE2(base_dtype, lo_dtype, BT, LT,
                     return launch_add<BT, LT>(base, base_row_stride, lo, lo_row_stride, out,
                                               out_row_stride, n_rows, n_cols, scaling, vec,
                                               static_cast<hipStream_t>(stream)));
  return QL_EDTYPE;
}

extern "C" uint32_t qlora_dropout_keep_threshold(float p) {
  return ql_philox::keep_threshold(p);
}

extern "C" int qlora_lora_dropout_scale_bits(const void* in, int64_t in_row_stride, void* out,
                                             int64_t out_row_stride, uint8_t* bits,
                                             int64_t bits_group_stride, int64_t n_rows,
                                             int64_t n_cols, int dtype, uint64_t seed, float p,
                                             float scale, ql_stream_t stream) {
  if (n_rows < 0 || n_cols < 0 || n_rows > UINT32_MAX || !(p > 0.0f) || !(p < 1.0f))
    return QL_EINVAL;
  if (dtype != QL_BF16 && dtype != QL_F16) return QL_EDTYPE;
  if (n_rows == 0 || n_cols == 0) return QL_OK;
  if (!in || !out || !bits) return QL_EINVAL;
  if (n_cols % 8 || bits_group_stride < n_cols || bits_group_stride % 8) return QL_ESHAPE;
  if (!rows_vec_ok(in, in_row_stride, dtype, n_cols) || !rows_vec_ok(out, out_row_stride, dtype, n_cols))
    return QL_EALIGN;
  const dim3 grid((unsigned)n_rows);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t thr = ql_philox::keep_threshold(p);
  using B = typename Elem<QL_BF16>::T;
  if (dtype == QL_BF16)
    hipLaunchKernelGGL((dropout_bits_kernel<QL_BF16, QL_BF16>), grid, dim3(kThreads), 0, s,
                       (const B*)in, in_row_stride, (B*)out, out_row_stride, bits,
                       bits_group_stride, n_cols, seed, thr, scale);
  else
    hipLaunchKernelGGL((dropout_bits_kernel<QL_F16, QL_F16>), grid, dim3(kThreads), 0, s,
                       (const B*)in, in_row_stride, (B*)out, out_row_stride, bits,
                       bits_group_stride, n_cols, seed, thr, scale);
  return ql_launch_status();
}

template <int DT, int G>
void launch_masked_add(void* dx, int64_t dx_rs, const void* du, int64_t du_rs, const void* A,
                       int64_t a_rs, const SlotBits& bits, int64_t bits_gs, int64_t M, int64_t K,
                       float scale, dim3 grid, int row_blocks, hipStream_t s) {
  if constexpr (G == 4)
    hipLaunchKernelGGL((up_masked_add4_kernel<DT>), grid, dim3(kThreads), 0, s, (uint16_t*)dx,
                       dx_rs, (const uint16_t*)du, du_rs, (const uint16_t*)A, a_rs, bits, bits_gs,
                       M, K, scale, row_blocks);
  else
    hipLaunchKernelGGL((up_masked_add_kernel<DT, G>), grid, dim3(kThreads), 0, s, (uint16_t*)dx,
                       dx_rs, (const uint16_t*)du, du_rs, (const uint16_t*)A, a_rs, bits, bits_gs,
                       M, K, scale, row_blocks);
}

template <int DT>
void launch_masked_add_g(int slots, void* dx, int64_t dx_rs, const void* du, int64_t du_rs,
                         const void* A, int64_t a_rs, const SlotBits& bits, int64_t bits_gs,
                         int64_t M, int64_t K, float scale, dim3 grid, int rows, hipStream_t s) {
  switch (slots) {
    case 1: launch_masked_add<DT, 1>(dx, dx_rs, du, du_rs, A, a_rs, bits, bits_gs, M, K, scale, grid, rows, s); break;
    case 2: launch_masked_add<DT, 2>(dx, dx_rs, du, du_rs, A, a_rs, bits, bits_gs, M, K, scale, grid, rows, s); break;
    case 3: launch_masked_add<DT, 3>(dx, dx_rs, du, du_rs, A, a_rs, bits, bits_gs, M, K, scale, grid, rows, s); break;
    default: launch_masked_add<DT, 4>(dx, dx_rs, du, du_rs, A, a_rs, bits, bits_gs, M, K, scale, grid, rows, s); break;
  }
}

extern "C" int qlora_lora_up_masked_add_slots(void* dx, int64_t dx_row_stride, const void* du,
                                              int64_t du_row_stride, const void* A,
                                              int64_t a_row_stride, const uint8_t* const* bits,
                                              int64_t bits_group_stride, int slots, int64_t M,
                                              int64_t K, int dtype, float scale,
                                              ql_stream_t stream) {
  if (M < 0 || K < 0 || slots < 1 || slots > 4) return QL_EINVAL;
  if (dtype != QL_BF16 && dtype != QL_F16) return QL_EDTYPE;
  if (M == 0 || K == 0) return QL_OK;
  if (!dx || !du || !A || !bits) return QL_EINVAL;
  SlotBits sb{};
  for (int g = 0; g < slots; ++g) {
    if (!bits[g]) return QL_EINVAL;
    sb.p[g] = bits[g];
  }
  if (K % 8 || bits_group_stride < K || bits_group_stride % 8 || du_row_stride < 16 * slots ||
      a_row_stride < K)
    return QL_ESHAPE;
  if (!rows_vec_ok(dx, dx_row_stride, dtype, K) || !rows_vec_ok(A, a_row_stride, dtype, K) ||
      !rows_vec_ok(du, du_row_stride, dtype, 16))
    return QL_EALIGN;
  const int64_t cols_per_block = (int64_t)(kThreads / 64) * kMaskedCols;
  const int64_t gx = (K + cols_per_block - 1) / cols_per_block;
  const int rows = 4;  // row blocks of 16 per workgroup
  const int64_t gy = (M + 16 * rows - 1) / (16 * rows);
  if (gx > INT32_MAX || gy > 65535) return QL_ESHAPE;
  const dim3 grid((unsigned)gx, (unsigned)gy);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == QL_BF16)
    launch_masked_add_g<QL_BF16>(slots, dx, dx_row_stride, du, du_row_stride, A, a_row_stride, sb,
                                 bits_group_stride, M, K, scale, grid, rows, s);
  else
    launch_masked_add_g<QL_F16>(slots, dx, dx_row_stride, du, du_row_stride, A, a_row_stride, sb,
                                bits_group_stride, M, K, scale, grid, rows, s);
  return ql_launch_status();
}

extern "C" int qlora_lora_up_masked_add(void* dx, int64_t dx_row_stride, const void* du,
                                        int64_t du_row_stride, const void* A, int64_t a_row_stride,
                                        const uint8_t* bits, int64_t bits_group_stride, int64_t M,
                                        int64_t K, int dtype, float scale, ql_stream_t stream) {
  if (!bits && M > 0 && K > 0) return QL_EINVAL;
  const uint8_t* one[1] = {bits};
  return qlora_lora_up_masked_add_slots(dx, dx_row_stride, du, du_row_stride, A, a_row_stride, one,
                                        bits_group_stride, 1, M, K, dtype, scale, stream);
}
