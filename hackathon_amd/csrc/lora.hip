// LoRA elementwise kernels around the adapter GEMMs, for gfx950.
//
// Reference semantics:
//   solution/lora.py:29-46  OUT = IN * keep * scale (keep from a counter-based RNG), or a
//                           plain scale-and-cast when dropout is off;
//   solution/lora.py:49-60  OUT = BASE + LO * scaling in fp32.
//
// The dropout mask is regenerated (never stored): keep = U(seed, row*N + col) > p, with U the
// uniform of Philox4x32-10 (Salmon et al., "Parallel Random Numbers: As Easy as 1, 2, 3",
// SC'11) on counter {flat index, 0, 0, 0} and key {seed_lo, seed_hi}; word 0 is folded to a
// non-negative int32 (x < 0 -> -x-1) and scaled by 4.6566127342e-10f. That is the uniform
// Triton's tl.rand(seed, int32 offset) draws, so a seed gives the reference's mask.
//
// HBM-bound. One workgroup per row; each thread moves 8 consecutive elements per step.
#include "ql_vec.h"

namespace {

constexpr int kThreads = 256;

// Each round's two 32 x 32 -> 64-bit products are written as 64-bit multiplies, so that each
// becomes one v_mad_u64_u32 instead of a v_mul_hi_u32 and a v_mul_lo_u32 (the 32-bit integer
// multiplies are the kernel's bound): 15% faster at 4096 x 3584, the same bits.
QL_DEV uint32_t philox_word0(uint32_t ctr, uint64_t seed) {
  uint32_t c0 = ctr, c1 = 0u, c2 = 0u, c3 = 0u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c0;
}

QL_DEV float uniform_from_word(uint32_t w) {
  int32_t x = (int32_t)w;
  x = x < 0 ? ~x : x;  // -x - 1 in two's complement, also for INT32_MIN
  return (float)x * 4.6566127342e-10f;
}

template <int IT, int OT, bool DROPOUT, bool VEC>
__global__ __launch_bounds__(kThreads) void dropout_scale_kernel(
    const typename Elem<IT>::T* __restrict__ in, int64_t in_rs, typename Elem<OT>::T* __restrict__ out,
    int64_t out_rs, int64_t n_cols, uint64_t seed, float p, float scale) {
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
          const bool keep = uniform_from_word(philox_word0(flat, seed)) > p;
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
        v = uniform_from_word(philox_word0(flat, seed)) > p ? v * scale : 0.0f;
      } else {
        v = v * scale;
      }
      dst[c] = Elem<OT>::from_f32(v);
    }
  }
}

// The dropout forward for the fused 4-bit LoRA layer: the same OUT = IN * keep * scale as
// dropout_scale_kernel (vector rows only), plus the keep mask as bits, byte c / 8 of row `row`
// holding columns c .. c + 7 (bit j = column c + j), so the backward needs no second Philox pass.
template <int IT, int OT>
__global__ __launch_bounds__(kThreads) void dropout_bits_kernel(
    const typename Elem<IT>::T* __restrict__ in, int64_t in_rs, typename Elem<OT>::T* __restrict__ out,
    int64_t out_rs, uint8_t* __restrict__ bits, int64_t bits_rs, int64_t n_cols, uint64_t seed,
    float p, float scale) {
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
      const bool keep = uniform_from_word(philox_word0(flat, seed)) > p;
      v[j] = keep ? v[j] * scale : 0.0f;
      b |= (uint32_t)keep << j;
    }
    Vec8<OT>::store(dst + c, v);
    bits[row * bits_rs + c / 8] = (uint8_t)b;
  }
}

// The dropout backward of G adapters' input gradients (the adapters of a group that read the
// same input, each with its own mask), added to the base gradient in one pass:
//   dx[m, k] += scale * sum_{g < G, keep_g(m, k)} sum_{r < 16} du[m, 16 g + r] * A[16 g + r, k]
// (du = s g B [M, >= 16 G], A [16 G, K] in dx's dtype; keep_g from adapter g's forward bits).
// Each rank-16 sum is 8 two-term dot products (v_dot2_f32_bf16 / _f16: exact 16-bit products
// summed in fp32) over r = 0 .. 15; the kept adapters' sums are added in fp32 in slot order and
// dx is rounded once (an element no adapter keeps is left as it is). Each thread owns CW
// consecutive columns, with A's pairs (A[16 g + 2i][k], A[16 g + 2i + 1][k]) in registers: 64
// of them a slot at CW = 8 (G <= 2), 32 at CW = 4 (G = 3, 4); and walks `rows` rows: 4 when the
// columns take at most 3 blocks of 256 threads (the grid stays large), else 16 (fewer reloads
// of A's pairs). Measured on MI355X at G = 1: 4096 x 3584 15.6 us (16 rows: 16.6), 4096 x 18944
// 77.6 us (4 rows: 92.7).

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2_t;

template <int DT> QL_DEV float dot2_acc(uint32_t a, uint32_t b, float c);
template <> QL_DEV float dot2_acc<QL_BF16>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}
template <> QL_DEV float dot2_acc<QL_F16>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c,
                                false);
}

// CW consecutive 16-bit values of a row as floats (CW = 8: one 16-B access, CW = 4: 8 B).
template <int DT, int CW> struct Cols;
template <int DT> struct Cols<DT, 8> {
  static QL_DEV void words(const uint16_t* p, uint32_t* w) {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    w[0] = r.x; w[1] = r.y; w[2] = r.z; w[3] = r.w;
  }
  static QL_DEV void load(const uint16_t* p, float* v) { Vec8<DT>::load(p, v); }
  static QL_DEV void store(uint16_t* p, const float* v) { Vec8<DT>::store(p, v); }
};
template <int DT> struct Cols<DT, 4> {
  static QL_DEV void words(const uint16_t* p, uint32_t* w) {
    const uint2 r = *reinterpret_cast<const uint2*>(p);
    w[0] = r.x; w[1] = r.y;
  }
  static QL_DEV void load(const uint16_t* p, float* v) {
    const uint2 r = *reinterpret_cast<const uint2*>(p);
    float t[8];
    Vec8<DT>::unpack(make_uint4(r.x, r.y, 0u, 0u), t);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = t[j];
  }
  static QL_DEV void store(uint16_t* p, const float* v) {
    const float t[8] = {v[0], v[1], v[2], v[3], 0.f, 0.f, 0.f, 0.f};
    const uint4 r = Vec8<DT>::pack(t);
    *reinterpret_cast<uint2*>(p) = make_uint2(r.x, r.y);
  }
};

struct SlotBits {
  const uint8_t* p[4];  // adapter g's keep bits [M, >= K / 8], one row stride for all
};

template <int DT, int G, int CW>
__global__ __launch_bounds__(kThreads) void up_masked_add_kernel(
    typename Elem<DT>::T* __restrict__ dx, int64_t dx_rs, const typename Elem<DT>::T* __restrict__ du,
    int64_t du_rs, const typename Elem<DT>::T* __restrict__ A, int64_t a_rs, SlotBits bits,
    int64_t bits_rs, int64_t M, int64_t K, float scale, int rows) {
#pragma clang fp contract(off)
  const int64_t c = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * CW;
  if (c >= K) return;
  uint32_t ap[G][8][CW];  // [slot][pair i][column j]: A[16 g + 2i][c + j] low, A[.. + 1] high
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t lw[CW / 2], hw[CW / 2];
      Cols<DT, CW>::words(A + (16 * g + 2 * i) * a_rs + c, lw);
      Cols<DT, CW>::words(A + (16 * g + 2 * i + 1) * a_rs + c, hw);
#pragma unroll
      for (int w = 0; w < CW / 2; ++w) {
        ap[g][i][2 * w] = __builtin_amdgcn_perm(hw[w], lw[w], 0x05040100u);
        ap[g][i][2 * w + 1] = __builtin_amdgcn_perm(hw[w], lw[w], 0x07060302u);
      }
    }
  const int shift = (int)(c & 7);  // 0, or 4 for the second half-byte at CW = 4
  const int64_t m0 = (int64_t)blockIdx.y * rows;
  const int64_t m1 = m0 + rows < M ? m0 + rows : M;
  for (int64_t m = m0; m < m1; ++m) {
    float v[CW], sum[CW] = {};
    uint32_t kept = 0;
    Cols<DT, CW>::load(dx + m * dx_rs + c, v);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint4 d0 = *reinterpret_cast<const uint4*>(du + m * du_rs + 16 * g);
      const uint4 d1 = *reinterpret_cast<const uint4*>(du + m * du_rs + 16 * g + 8);
      const uint32_t dp[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
      const uint32_t b = (uint32_t)bits.p[g][m * bits_rs + c / 8] >> shift;
#pragma unroll
      for (int j = 0; j < CW; ++j) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) t = dot2_acc<DT>(dp[i], ap[g][i][j], t);
        if ((b >> j) & 1u) {
          sum[j] = (kept >> j) & 1u ? sum[j] + t : t;
          kept |= 1u << j;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < CW; ++j)
      if ((kept >> j) & 1u) v[j] = v[j] + scale * sum[j];
    Cols<DT, CW>::store(dx + m * dx_rs + c, v);
  }
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
                     (const I*)in, in_rs, (O*)out, out_rs, n_cols, seed, p, scale)
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

extern "C" int qlora_lora_dropout_scale_bits(const void* in, int64_t in_row_stride, void* out,
                                             int64_t out_row_stride, uint8_t* bits,
                                             int64_t bits_row_stride, int64_t n_rows,
                                             int64_t n_cols, int dtype, uint64_t seed, float p,
                                             float scale, ql_stream_t stream) {
  if (n_rows < 0 || n_cols < 0 || n_rows > UINT32_MAX || !(p > 0.0f) || !(p < 1.0f))
    return QL_EINVAL;
  if (dtype != QL_BF16 && dtype != QL_F16) return QL_EDTYPE;
  if (n_rows == 0 || n_cols == 0) return QL_OK;
  if (!in || !out || !bits) return QL_EINVAL;
  if (n_cols % 8 || bits_row_stride < n_cols / 8) return QL_ESHAPE;
  if (!rows_vec_ok(in, in_row_stride, dtype, n_cols) || !rows_vec_ok(out, out_row_stride, dtype, n_cols))
    return QL_EALIGN;
  const dim3 grid((unsigned)n_rows);
  hipStream_t s = static_cast<hipStream_t>(stream);
  using B = typename Elem<QL_BF16>::T;
  if (dtype == QL_BF16)
    hipLaunchKernelGGL((dropout_bits_kernel<QL_BF16, QL_BF16>), grid, dim3(kThreads), 0, s,
                       (const B*)in, in_row_stride, (B*)out, out_row_stride, bits,
                       bits_row_stride, n_cols, seed, p, scale);
  else
    hipLaunchKernelGGL((dropout_bits_kernel<QL_F16, QL_F16>), grid, dim3(kThreads), 0, s,
                       (const B*)in, in_row_stride, (B*)out, out_row_stride, bits,
                       bits_row_stride, n_cols, seed, p, scale);
  return ql_launch_status();
}

template <int DT, int G>
void launch_masked_add(void* dx, int64_t dx_rs, const void* du, int64_t du_rs, const void* A,
                       int64_t a_rs, const SlotBits& bits, int64_t bits_rs, int64_t M, int64_t K,
                       float scale, dim3 grid, int rows, hipStream_t s) {
  constexpr int CW = G <= 2 ? 8 : 4;
  using T = typename Elem<DT>::T;
  hipLaunchKernelGGL((up_masked_add_kernel<DT, G, CW>), grid, dim3(kThreads), 0, s, (T*)dx, dx_rs,
                     (const T*)du, du_rs, (const T*)A, a_rs, bits, bits_rs, M, K, scale, rows);
}

template <int DT>
void launch_masked_add_g(int slots, void* dx, int64_t dx_rs, const void* du, int64_t du_rs,
                         const void* A, int64_t a_rs, const SlotBits& bits, int64_t bits_rs,
                         int64_t M, int64_t K, float scale, dim3 grid, int rows, hipStream_t s) {
  switch (slots) {
    case 1: launch_masked_add<DT, 1>(dx, dx_rs, du, du_rs, A, a_rs, bits, bits_rs, M, K, scale, grid, rows, s); break;
    case 2: launch_masked_add<DT, 2>(dx, dx_rs, du, du_rs, A, a_rs, bits, bits_rs, M, K, scale, grid, rows, s); break;
    case 3: launch_masked_add<DT, 3>(dx, dx_rs, du, du_rs, A, a_rs, bits, bits_rs, M, K, scale, grid, rows, s); break;
    default: launch_masked_add<DT, 4>(dx, dx_rs, du, du_rs, A, a_rs, bits, bits_rs, M, K, scale, grid, rows, s); break;
  }
}

extern "C" int qlora_lora_up_masked_add_slots(void* dx, int64_t dx_row_stride, const void* du,
                                              int64_t du_row_stride, const void* A,
                                              int64_t a_row_stride, const uint8_t* const* bits,
                                              int64_t bits_row_stride, int slots, int64_t M,
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
  if (K % 8 || bits_row_stride < K / 8 || du_row_stride < 16 * slots || a_row_stride < K)
    return QL_ESHAPE;
  if (!rows_vec_ok(dx, dx_row_stride, dtype, K) || !rows_vec_ok(A, a_row_stride, dtype, K) ||
      !rows_vec_ok(du, du_row_stride, dtype, 16))
    return QL_EALIGN;
  const int cw = slots <= 2 ? 8 : 4;
  const int64_t gx = (K / cw + kThreads - 1) / kThreads;
  const int rows = gx <= 3 ? 4 : 16;
  const int64_t gy = (M + rows - 1) / rows;
  if (gx > INT32_MAX || gy > 65535) return QL_ESHAPE;
  const dim3 grid((unsigned)gx, (unsigned)gy);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == QL_BF16)
    launch_masked_add_g<QL_BF16>(slots, dx, dx_row_stride, du, du_row_stride, A, a_row_stride, sb,
                                 bits_row_stride, M, K, scale, grid, rows, s);
  else
    launch_masked_add_g<QL_F16>(slots, dx, dx_row_stride, du, du_row_stride, A, a_row_stride, sb,
                                bits_row_stride, M, K, scale, grid, rows, s);
  return ql_launch_status();
}

extern "C" int qlora_lora_up_masked_add(void* dx, int64_t dx_row_stride, const void* du,
                                        int64_t du_row_stride, const void* A, int64_t a_row_stride,
                                        const uint8_t* bits, int64_t bits_row_stride, int64_t M,
                                        int64_t K, int dtype, float scale, ql_stream_t stream) {
  if (!bits && M > 0 && K > 0) return QL_EINVAL;
  const uint8_t* one[1] = {bits};
  return qlora_lora_up_masked_add_slots(dx, dx_row_stride, du, du_row_stride, A, a_row_stride, one,
                                        bits_row_stride, 1, M, K, dtype, scale, stream);
}
