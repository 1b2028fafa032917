// Rank-16 LoRA contractions on CDNA4 matrix cores, for gfx950.
//
// The adapter GEMMs of a LoRA layer (the nn.Linear pair of solution/lora.py:172 and what
// autograd computes for it) are skinny: one side is the rank r = 16. As plain GEMMs they
// leave most of the GPU idle (a 4096 x 16 output is 32 tiles of 128 x 128). Two kernels
// cover them, both streaming the large operand from HBM exactly once:
//
//   lora_down   out[m, c] = alpha * sum_k X[m, k] * Y[c, k]        (c < 16)
//               u = x A^T (forward) and du = s * g B (backward, Y = B^T): X [M, K]
//               k-contiguous, Y [16, K] k-contiguous. Output bf16/fp16 [M, ldo] with
//               columns 16 .. out_cols-1 zero-filled, so it can serve as the extra
//               K = 64 segment of the base GEMM.
//   lora_wgrad  out[n, c] = alpha * sum_m Q[m, n] * P[m, c]        (c < 16), fp32 [N, 16]
//               dB = s * g^T u and dA^T = x^T du: the reduction runs over the token rows,
//               which are the strided dimension of both operands.
//
// lora_down: one workgroup (4 waves) per 16 rows and K range. A v_mfma_f32_16x16x32 needs
// 8 consecutive k per lane; the sum over k does not care which 8, so for MFMA t of a 128-k
// chunk lane l supplies k = 32 t + 8 (l/16) .. +7 of row l%16: each 16-B load instruction
// then reads 64 contiguous bytes from each of 16 rows. Y is read with the same k map. Waves
// take alternate 128-k chunks and are summed through LDS.
//
// lora_wgrad: one workgroup per 128 columns and M range. Lane l loads an 8 (rows) x 8
// (columns) block of Q as eight 16-B row pieces (lanes 0-15 of a row read 256 contiguous
// bytes), transposes it in registers with byte permutes into eight fragments that each hold
// 8 consecutive rows of one column, and multiplies them by the fragment of P for the same 8
// rows: MFMA t accumulates columns n0 + 8*(l%16) + t. Waves take alternate 32-row chunks and
// are summed through LDS.
//
// Both kernels optionally split their reduction over blockIdx.y into an fp32 workspace,
// summed in split order by the matching reduce kernel (deterministic).
#include "ql_vec.h"
#include "lora_mfma.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

constexpr int kThreads = 256;
constexpr int kRank = 16;

template <int DT> QL_DEV f32x4_t mfma(const uint4& a, const uint4& b, f32x4_t c);
template <> QL_DEV f32x4_t mfma<QL_BF16>(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <> QL_DEV f32x4_t mfma<QL_F16>(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Sum a per-lane f32x4 over the 4 waves of the workgroup; the result is valid in wave 0.
QL_DEV f32x4_t wave_reduce4(f32x4_t v, f32x4_t* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  red[wave * 64 + lane] = v;
  __syncthreads();
  f32x4_t s = red[lane];
#pragma unroll
  for (int w = 1; w < 4; ++w) s += red[w * 64 + lane];
  __syncthreads();
  return s;
}

// ---------------------------------------------------------------------------------------
constexpr int kDownUnroll = 4;  // 128-k chunks per wave in flight (16 x 16-B loads per lane)
constexpr int kDownWaves = 8;   // two waves per SIMD: twice the loads in flight per CU

// Sum a per-lane f32x4 over the kDownWaves waves of the workgroup; valid in wave 0.
QL_DEV f32x4_t wave_reduce_n(f32x4_t v, f32x4_t* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  red[wave * 64 + lane] = v;
  __syncthreads();
  f32x4_t s = red[lane];
#pragma unroll
  for (int w = 1; w < kDownWaves; ++w) s += red[w * 64 + lane];
  return s;
}

template <int IT, int OT, bool PARTIAL>
__global__ __launch_bounds__(64 * kDownWaves) void lora_down_kernel(
    const uint16_t* __restrict__ X, int64_t ldx, const uint16_t* __restrict__ Y, int64_t ldy,
    int64_t M, int64_t K, int64_t k_per_split, float* __restrict__ ws,
    typename Elem<OT>::T* __restrict__ out, int64_t ldo, int out_cols, float alpha,
    uint16_t* __restrict__ out_t, int64_t ldt) {
  __shared__ f32x4_t red[kDownWaves * 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m0 = (int64_t)blockIdx.x * 16;
  const int64_t row = m0 + (lane & 15);
  const int64_t rowc = row < M ? row : M - 1;
  const int64_t kb = (int64_t)blockIdx.y * k_per_split;
  const int64_t ke = kb + k_per_split < K ? kb + k_per_split : K;
  const int koff = 8 * (lane >> 4);
  const uint16_t* xr = X + rowc * ldx;
  const uint16_t* yr = Y + (int64_t)(lane & 15) * ldy;
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  // Wave w takes the 128-k chunks w, w + 8, w + 16, ... (slots j = 0 .. J-1) of its K range,
  // kDownUnroll at a time, starting at slot (blockIdx.x mod J): workgroups running at the
  // same time then read different parts of Y, which every workgroup reads whole, instead of
  // all asking the same L2 lines at once. MFMA t of a chunk takes k = chunk + 32 t +
  // 8 (lane / 16) .. +7: each load instruction reads 64 contiguous bytes of each of the 16
  // rows. K and every chunk start are multiples of 32, so a 32-k group is all in or all out;
  // groups past the end load an in-range address and contribute zeros (the MFMAs below must
  // run with every lane's operands defined, so nothing here is under a lane-dependent branch).
  constexpr int64_t kStride = 128 * kDownWaves;
  const int64_t J = (ke - kb + kStride - 1) / kStride;
  const int64_t rot = J > 0 ? (int64_t)blockIdx.x % J : 0;
  for (int64_t j0 = 0; j0 < J; j0 += kDownUnroll) {  // uniform per workgroup
    uint4 xv[kDownUnroll][4], yv[kDownUnroll][4];
#pragma unroll
    for (int u = 0; u < kDownUnroll; ++u) {
      const uint4 z = make_uint4(0, 0, 0, 0);
      if (j0 + u >= J) {  // workgroup-uniform: no slot left, no loads
#pragma unroll
        for (int t = 0; t < 4; ++t) xv[u][t] = yv[u][t] = z;
        continue;
      }
      int64_t js = j0 + u + rot;
      js = js >= J ? js - J : js;
      const int64_t c0 = kb + 128 * wave + kStride * js;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int64_t k = c0 + 32 * t;
        const bool ok = k < ke;
        const int64_t kk = (ok ? k : kb) + koff;
        const uint4 xr4 = *reinterpret_cast<const uint4*>(xr + kk);
        const uint4 yr4 = *reinterpret_cast<const uint4*>(yr + kk);
        xv[u][t] = ok ? xr4 : z;
        yv[u][t] = ok ? yr4 : z;
      }
    }
#pragma unroll
    for (int u = 0; u < kDownUnroll; ++u) {
      acc0 = mfma<IT>(yv[u][0], xv[u][0], acc0);
      acc1 = mfma<IT>(yv[u][1], xv[u][1], acc1);
      acc0 = mfma<IT>(yv[u][2], xv[u][2], acc0);
      acc1 = mfma<IT>(yv[u][3], xv[u][3], acc1);
    }
  }
  const f32x4_t s = wave_reduce_n(acc0 + acc1, red);
  if (wave != 0 || row >= M) return;
  // lane holds out[row][c .. c+3], c = 4 * (lane / 16)
  const int c = 4 * (lane >> 4);
  if constexpr (PARTIAL) {
    *reinterpret_cast<float4*>(ws + ((int64_t)blockIdx.y * M + row) * kRank + c) =
        make_float4(s[0], s[1], s[2], s[3]);
  } else {
    auto* o = out + row * ldo;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[c + e] = Elem<OT>::from_f32(alpha * s[e]);
    for (int z = kRank + c; z < out_cols; z += 16)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (z + e < out_cols) o[z + e] = Elem<OT>::from_f32(0.f);
    if (out_t) {  // [16, M]: the 16 lanes of a row group write 32 contiguous bytes per c
#pragma unroll
      for (int e = 0; e < 4; ++e)
        out_t[(int64_t)(c + e) * ldt + row] = Elem<IT>::from_f32(alpha * s[e]);
    }
  }
}

template <int IT, int OT>
__global__ __launch_bounds__(256) void lora_down_reduce(const float* __restrict__ ws, int splits,
                                                        int64_t M, typename Elem<OT>::T* __restrict__ out,
                                                        int64_t ldo, int out_cols, float alpha,
                                                        uint16_t* __restrict__ out_t, int64_t ldt) {
  const int64_t total = M * out_cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / out_cols;
    const int c = (int)(i - m * out_cols);
    float v = 0.f;
    if (c < kRank) {
      // 8 partials loaded at a time, added in split order
      const float* wp = ws + m * kRank + c;
      const int64_t stride = M * kRank;
      int z = 0;
      for (; z + 8 <= splits; z += 8) {
        float w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = wp[(int64_t)(z + j) * stride];
#pragma unroll
        for (int j = 0; j < 8; ++j) v += w[j];
      }
      for (; z < splits; ++z) v += wp[(int64_t)z * stride];
      v *= alpha;
      if (out_t) out_t[(int64_t)c * ldt + m] = Elem<IT>::from_f32(v);
    }
    out[m * ldo + c] = Elem<OT>::from_f32(v);
  }
}

// ---------------------------------------------------------------------------------------
// 8 x 8 transpose of 16-bit values: in[i] holds row i (8 columns as 4 words, column pairs);
// out[t] holds column t (8 rows as 4 words, row pairs).
QL_DEV void transpose8x8(const uint4 (&in)[8], uint4 (&out)[8]) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint4& r0 = in[2 * p];
      const uint4& r1 = in[2 * p + 1];
      const uint32_t a = (t >> 1) == 0 ? r0.x : (t >> 1) == 1 ? r0.y : (t >> 1) == 2 ? r0.z : r0.w;
      const uint32_t b = (t >> 1) == 0 ? r1.x : (t >> 1) == 1 ? r1.y : (t >> 1) == 2 ? r1.z : r1.w;
      // even column: low halves of a and b; odd column: high halves
      w[p] = (t & 1) ? __builtin_amdgcn_perm(b, a, 0x07060302u)
                     : __builtin_amdgcn_perm(b, a, 0x05040100u);
    }
    out[t] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

constexpr int kWgradUnroll = 4;  // 32-row chunks per wave in flight

// Store 4 consecutive values (n, c .. c+3) of out [N, 16] (or of its transpose [16, N]).
QL_DEV void store_wgrad4(float* __restrict__ out, bool out_t, int64_t N, int64_t n, int64_t c,
                         float4 v) {
  if (out_t) {
    out[(c + 0) * N + n] = v.x;
    out[(c + 1) * N + n] = v.y;
    out[(c + 2) * N + n] = v.z;
    out[(c + 3) * N + n] = v.w;
  } else {
    *reinterpret_cast<float4*>(out + n * kRank + c) = v;
  }
}

// PARTIAL: each split writes its fp32 [N, 16] partial to ws[split]; lora_wgrad_reduce sums
// them in split order. (Summing inside this launch by the last workgroup of each column block
// needs device-scope release/acquire fences per workgroup, whose L2 write-back and invalidate
// cost more than the separate reduce launch.)
template <int IT, bool PARTIAL>
__global__ __launch_bounds__(kThreads) void lora_wgrad_kernel(
    const uint16_t* __restrict__ PT, int64_t ldpt, const uint16_t* __restrict__ Q, int64_t ldq,
    int64_t M, int64_t N, int64_t m_per_split, float* __restrict__ ws, float* __restrict__ out,
    float alpha, bool out_t) {
  __shared__ f32x4_t red[4 * 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cg = lane & 15;                 // column group: columns n0 + 8 cg .. +7
  const int mq = lane >> 4;                 // rows 8 mq .. 8 mq + 7 of a 32-row chunk
  const int64_t n0 = (int64_t)blockIdx.x * 128;
  const int64_t ncol = n0 + 8 * cg;
  const bool col_ok = ncol < N;             // N % 8 == 0: a group is all in or all out
  const int64_t mb = (int64_t)blockIdx.y * m_per_split;
  const int64_t me = mb + m_per_split < M ? mb + m_per_split : M;
  const uint16_t* ptr_c = PT + (int64_t)cg * ldpt;  // row cg of P^T: P[:, cg], m-contiguous
  f32x4_t acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int64_t m = mb + 32 * wave; m < me; m += 128 * kWgradUnroll) {  // uniform per wave
    uint4 q[kWgradUnroll][8], pf[kWgradUnroll];
#pragma unroll
    for (int u = 0; u < kWgradUnroll; ++u) {
      const int64_t r0 = m + 128 * u + 8 * mq;
      if (r0 + 8 <= me) {
        pf[u] = *reinterpret_cast<const uint4*>(ptr_c + r0);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          q[u][i] = col_ok ? *reinterpret_cast<const uint4*>(Q + (r0 + i) * ldq + ncol)
                           : make_uint4(0, 0, 0, 0);
      } else {  // rows past the range contribute zeros
        uint16_t pv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const bool ok = r0 + i < me;
          pv[i] = ok ? ptr_c[r0 + i] : (uint16_t)0;
          q[u][i] = (ok && col_ok) ? *reinterpret_cast<const uint4*>(Q + (r0 + i) * ldq + ncol)
                                   : make_uint4(0, 0, 0, 0);
        }
        pf[u] = make_uint4((uint32_t)pv[0] | ((uint32_t)pv[1] << 16),
                           (uint32_t)pv[2] | ((uint32_t)pv[3] << 16),
                           (uint32_t)pv[4] | ((uint32_t)pv[5] << 16),
                           (uint32_t)pv[6] | ((uint32_t)pv[7] << 16));
      }
    }
#pragma unroll
    for (int u = 0; u < kWgradUnroll; ++u) {
      uint4 qt[8];
      transpose8x8(q[u], qt);
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] = mfma<IT>(pf[u], qt[t], acc[t]);
    }
  }
  // acc[t]: lane holds out[n = n0 + 8*(lane%16) + t][c = 4*(lane/16) .. +3]
  const int c = 4 * (lane >> 4);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const f32x4_t s = wave_reduce4(acc[t], red);
    if (wave == 0 && col_ok) {
      const int64_t n = ncol + t;
      if constexpr (PARTIAL) {
        *reinterpret_cast<float4*>(ws + ((int64_t)blockIdx.y * N + n) * kRank + c) =
            make_float4(s[0], s[1], s[2], s[3]);
      } else {
        store_wgrad4(out, out_t, N, n, c,
                     make_float4(alpha * s[0], alpha * s[1], alpha * s[2], alpha * s[3]));
      }
    }
  }
}

// out = alpha * sum over splits of ws[split] ([N, 16] fp32 each), in split order; one thread
// per 4 consecutive values. splits = 0 writes zeros.
__global__ __launch_bounds__(256) void lora_wgrad_reduce(const float* __restrict__ ws, int splits,
                                                         int64_t N, float* __restrict__ out,
                                                         float alpha, bool out_t) {
  const int64_t total4 = N * kRank / 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total4;
       i += (int64_t)gridDim.x * 256) {
    // 8 partials loaded at a time (independent loads in flight), added in split order
    const float4* w4 = reinterpret_cast<const float4*>(ws) + i;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    int z = 0;
    for (; z + 8 <= splits; z += 8) {
      float4 w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) w[j] = w4[(int64_t)(z + j) * total4];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v.x += w[j].x; v.y += w[j].y; v.z += w[j].z; v.w += w[j].w;
      }
    }
    for (; z < splits; ++z) {
      const float4 w = w4[(int64_t)z * total4];
      v.x += w.x; v.y += w.y; v.z += w.z; v.w += w.w;
    }
    const int64_t n = (4 * i) / kRank, c = 4 * i - n * kRank;
    store_wgrad4(out, out_t, N, n, c, make_float4(alpha * v.x, alpha * v.y, alpha * v.z,
                                                  alpha * v.w));
  }
}

// ---------------------------------------------------------------------------------------
// The compute-dtype forms of one adapter's fp32 factors A [16, K] and B [N, 16], in one pass:
//   a16 [16, K]  = A                    (the Y operand of u = x A^T)
//   at  [K, 64]  = A^T | 0              (the second K segment of the backward dX GEMM)
//   bs  [N, 64]  = s B | 0              (the second K segment of the forward GEMM)
//   bt  [16, N]  = B^T                  (the Y operand of du = s g B)
// Thread t of the flat range handles one row of at (t < K), then one row of bs and one
// column of bt (K <= t < K + N), then 8 elements of a16.
template <int OT>
__global__ __launch_bounds__(256) void lora_pack_kernel(const float* __restrict__ A,
                                                        const float* __restrict__ B, int64_t K,
                                                        int64_t N, float scaling,
                                                        typename Elem<OT>::T* __restrict__ a16,
                                                        typename Elem<OT>::T* __restrict__ at,
                                                        typename Elem<OT>::T* __restrict__ bs,
                                                        typename Elem<OT>::T* __restrict__ bt,
                                                        int pad) {
  using T = typename Elem<OT>::T;
  const int64_t n_a16 = kRank * K / 8;
  const int64_t total = K + N + n_a16;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * 256) {
    if (t < K) {
      T* row = at + t * pad;
#pragma unroll
      for (int r = 0; r < kRank; ++r) row[r] = Elem<OT>::from_f32(A[(int64_t)r * K + t]);
      for (int c = kRank; c < pad; ++c) row[c] = Elem<OT>::from_f32(0.f);
    } else if (t < K + N) {
      const int64_t n = t - K;
      T* row = bs + n * pad;
#pragma unroll
      for (int r = 0; r < kRank; ++r) {
        const float b = B[n * kRank + r];
        row[r] = Elem<OT>::from_f32(scaling * b);
        bt[(int64_t)r * N + n] = Elem<OT>::from_f32(b);
      }
      for (int c = kRank; c < pad; ++c) row[c] = Elem<OT>::from_f32(0.f);
    } else {
      const int64_t i = (t - K - N) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) a16[i + e] = Elem<OT>::from_f32(A[i + e]);
    }
  }
}

// The compute-dtype operands of up to four rank-16 adapters that share an input (the q/k/v or
// gate/up projections of one layer) for one fused GEMM per direction: adapter g owns columns
// 16g .. 16g+15 of the padded operands and rows off[g] .. off[g+1]-1 of the concatenated
// outputs. Work items: t < K: row t of at (all pad columns); K <= t < K + N: row n of bs and
// column n of bt; then 8 elements of a16 per item.
constexpr int kMaxGroup = 4;
struct PackGroupArgs {
  const float* A[kMaxGroup];  // [16, K]
  const float* B[kMaxGroup];  // [n_g, 16]
  float scale[kMaxGroup];
  int64_t off[kMaxGroup + 1];  // prefix sums of n_g
  int G;
};

template <int OT>
__global__ __launch_bounds__(256) void lora_pack_group_kernel(PackGroupArgs p, int64_t K,
                                                              typename Elem<OT>::T* __restrict__ a16,
                                                              typename Elem<OT>::T* __restrict__ at,
                                                              typename Elem<OT>::T* __restrict__ bs,
                                                              typename Elem<OT>::T* __restrict__ bt,
                                                              int pad) {
  using T = typename Elem<OT>::T;
  const int64_t N = p.off[p.G];
  const int64_t n_a16 = (int64_t)kRank * p.G * K / 8;
  const int64_t total = K + N + n_a16;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * 256) {
    if (t < K) {
      // row t of at: 8 columns (one 16-B store) at a time
      T* row = at + t * pad;
      for (int c0 = 0; c0 < pad; c0 += 8) {
        const int g = c0 / kRank;
        float v[8];
        if (g < p.G) {
          const float* a = p.A[g] + (int64_t)(c0 & (kRank - 1)) * K + t;
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = a[(int64_t)e * K];
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = 0.f;
        }
        Vec8<OT>::store(row + c0, v);
      }
    } else if (t < K + N) {
      const int64_t n = t - K;
      int g = 0;
      while (g + 1 < p.G && n >= p.off[g + 1]) ++g;
      const int64_t ln = n - p.off[g];
      T* row = bs + n * pad;
      float b[kRank];
#pragma unroll
      for (int r = 0; r < kRank; ++r) {
        b[r] = p.B[g][ln * kRank + r];
        bt[(int64_t)r * N + n] = Elem<OT>::from_f32(b[r]);
      }
      for (int c0 = 0; c0 < pad; c0 += 8) {
        float v[8];
        const bool mine = c0 / kRank == g;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = mine ? p.scale[g] * b[(c0 & (kRank - 1)) + e] : 0.f;
        Vec8<OT>::store(row + c0, v);
      }
    } else {
      const int64_t i = (t - K - N) * 8;  // into a16 [16 G, K]
      const int64_t gr = i / K, col = i - gr * K;
      const int g = (int)(gr / kRank), r = (int)(gr - (int64_t)g * kRank);
#pragma unroll
      for (int e = 0; e < 8; ++e) a16[i + e] = Elem<OT>::from_f32(p.A[g][(int64_t)r * K + col + e]);
    }
  }
}

unsigned grid1d(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 4096) g = 4096;
  return (unsigned)(g > 0 ? g : 1);
}

}  // namespace

// ---- host side -------------------------------------------------------------------------

// Split K only while there are fewer than 256 row groups (one workgroup per CU is enough to
// stream X at full bandwidth with kDownUnroll chunks in flight per wave).
int ql_lora_down_splits(int64_t M, int64_t K) {
  const int64_t groups = (M + 15) / 16;
  int s = 1;
  while (groups * s < 256 && K / (128 * kDownWaves * 2 * s) >= 1 && s < 64) s *= 2;
  return s;
}

int64_t ql_lora_down_workspace_floats(int64_t M, int64_t K) {
  const int s = ql_lora_down_splits(M, K);
  return s > 1 ? (int64_t)s * M * kRank : 0;
}

int ql_lora_down(int in_dtype, int out_dtype, const void* X, int64_t ldx, const void* Y,
                 int64_t ldy, int64_t M, int64_t K, void* out, int64_t ldo, int out_cols,
                 float alpha, void* out_t, int64_t ldt, float* ws, int64_t ws_floats,
                 hipStream_t s) {
  if (M <= 0 || K <= 0 || K % 32 || out_cols < kRank || ldo < out_cols) return QL_EINVAL;
  if (out_t && ldt < M) return QL_EINVAL;
  if (ldx % 8 || ldy % 8 || !ql_aligned(X, 16) || !ql_aligned(Y, 16)) return QL_EALIGN;
  if (in_dtype != QL_BF16 && in_dtype != QL_F16) return QL_EDTYPE;
  if (out_dtype != QL_BF16 && out_dtype != QL_F16 && out_dtype != QL_F32) return QL_EDTYPE;
  int splits = ql_lora_down_splits(M, K);
  if (ws_floats < (int64_t)splits * M * kRank || !ws) splits = 1;
  // per-split K range: a multiple of 128 k per wave
  constexpr int64_t kq = 128 * kDownWaves;
  int64_t kps = ((K + splits - 1) / splits + kq - 1) / kq * kq;
  splits = (int)((K + kps - 1) / kps);
  const dim3 grid((unsigned)((M + 15) / 16), (unsigned)splits);
#define QL_DOWN(IT, OT)                                                                      \
  do {                                                                                       \
    using T = typename Elem<OT>::T;                                                          \
    if (splits == 1) {                                                                       \
      hipLaunchKernelGGL((lora_down_kernel<IT, OT, false>), grid, dim3(64 * kDownWaves), 0, s, \
                         (const uint16_t*)X, ldx, (const uint16_t*)Y, ldy, M, K, kps,        \
                         (float*)nullptr, (T*)out, ldo, out_cols, alpha, (uint16_t*)out_t,   \
                         ldt);                                                               \
    } else {                                                                                 \
      hipLaunchKernelGGL((lora_down_kernel<IT, OT, true>), grid, dim3(64 * kDownWaves), 0, s,  \
                         (const uint16_t*)X, ldx, (const uint16_t*)Y, ldy, M, K, kps, ws,    \
                         (T*)out, ldo, out_cols, alpha, (uint16_t*)out_t, ldt);              \
      hipLaunchKernelGGL((lora_down_reduce<IT, OT>), dim3(grid1d(M * out_cols)), dim3(256),  \
                         0, s, ws, splits, M, (T*)out, ldo, out_cols, alpha,                 \
                         (uint16_t*)out_t, ldt);                                             \
    }                                                                                        \
  } while (0)
  if (in_dtype == QL_BF16) {
    if (out_dtype == QL_BF16) QL_DOWN(QL_BF16, QL_BF16);
    else if (out_dtype == QL_F16) QL_DOWN(QL_BF16, QL_F16);
    else QL_DOWN(QL_BF16, QL_F32);
  } else {
    if (out_dtype == QL_BF16) QL_DOWN(QL_F16, QL_BF16);
    else if (out_dtype == QL_F16) QL_DOWN(QL_F16, QL_F16);
    else QL_DOWN(QL_F16, QL_F32);
  }
#undef QL_DOWN
  return ql_launch_status();
}

// Split the token range until there are at least 256 workgroups, keeping at least one
// 32-row chunk per wave in each split.
int ql_lora_wgrad_splits(int64_t M, int64_t N) {
  const int64_t blocks = (N + 127) / 128;
  int s = 1;
  while (blocks * s < 256 && M / (128 * 2 * s) >= 1 && s < 64) s *= 2;
  return s;
}

int64_t ql_lora_wgrad_workspace_floats(int64_t M, int64_t N) {
  const int s = ql_lora_wgrad_splits(M, N);
  return s > 1 ? (int64_t)s * N * kRank : 0;
}

int ql_lora_wgrad(int in_dtype, const void* PT, int64_t ldpt, const void* Q, int64_t ldq,
                  int64_t M, int64_t N, float* out, int out_t, float alpha, float* ws,
                  int64_t ws_floats, hipStream_t s) {
  if (M <= 0 || N <= 0 || N % 8 || ldpt < M) return QL_EINVAL;
  if (ldq % 8 || ldpt % 8 || !ql_aligned(Q, 16) || !ql_aligned(PT, 16) || !ql_aligned(out, 16))
    return QL_EALIGN;
  if (out_t != 0 && out_t != 1) return QL_EINVAL;
  if (in_dtype != QL_BF16 && in_dtype != QL_F16) return QL_EDTYPE;
  int splits = ql_lora_wgrad_splits(M, N);
  if (ws_floats < (int64_t)splits * N * kRank || !ws) splits = 1;
  int64_t mps = ((M + splits - 1) / splits + 127) / 128 * 128;
  splits = (int)((M + mps - 1) / mps);
  const dim3 grid((unsigned)((N + 127) / 128), (unsigned)splits);
#define QL_WGRAD(IT)                                                                         \
  do {                                                                                       \
    if (splits == 1) {                                                                       \
      hipLaunchKernelGGL((lora_wgrad_kernel<IT, false>), grid, dim3(kThreads), 0, s,         \
                         (const uint16_t*)PT, ldpt, (const uint16_t*)Q, ldq, M, N, mps,      \
                         (float*)nullptr, out, alpha, out_t);                                \
    } else {                                                                                 \
      hipLaunchKernelGGL((lora_wgrad_kernel<IT, true>), grid, dim3(kThreads), 0, s,          \
                         (const uint16_t*)PT, ldpt, (const uint16_t*)Q, ldq, M, N, mps, ws,  \
                         out, alpha, out_t);                                                 \
      hipLaunchKernelGGL(lora_wgrad_reduce, dim3(grid1d(N * kRank)), dim3(256), 0, s, ws,    \
                         splits, N, out, alpha, out_t);                                      \
    }                                                                                        \
  } while (0)
  if (in_dtype == QL_BF16) QL_WGRAD(QL_BF16);
  else QL_WGRAD(QL_F16);
#undef QL_WGRAD
  return ql_launch_status();
}

// ---- C-ABI -------------------------------------------------------------------------------

extern "C" int64_t qlora_lora_down_workspace_size(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0) return 0;
  return ql_lora_down_workspace_floats(M, K) * (int64_t)sizeof(float);
}

extern "C" int qlora_lora_down(const void* X, int64_t ldx, const void* Y, int64_t ldy, int64_t M,
                               int64_t K, int in_dtype, void* out, int64_t ldo, int out_cols,
                               int out_dtype, float alpha, void* out_t, int64_t ldt,
                               void* workspace, int64_t workspace_bytes, ql_stream_t stream) {
  if (M < 0 || K < 0 || workspace_bytes < 0) return QL_EINVAL;
  if (M == 0) return QL_OK;
  if (!X || !Y || !out) return QL_EINVAL;
  if (workspace && !ql_aligned(workspace, 16)) return QL_EALIGN;
  if (out_t && !ql_aligned(out_t, 2)) return QL_EALIGN;
  return ql_lora_down(in_dtype, out_dtype, X, ldx, Y, ldy, M, K, out, ldo, out_cols, alpha,
                      out_t, ldt, static_cast<float*>(workspace),
                      workspace_bytes / (int64_t)sizeof(float),
                      static_cast<hipStream_t>(stream));
}

extern "C" int64_t qlora_lora_wgrad_workspace_size(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return 0;
  return ql_lora_wgrad_workspace_floats(M, N) * (int64_t)sizeof(float);
}

extern "C" int qlora_lora_wgrad(const void* PT, int64_t ldpt, const void* Q, int64_t ldq, int64_t M,
                                int64_t N, int in_dtype, float* out, int out_transposed,
                                float alpha, void* workspace, int64_t workspace_bytes,
                                ql_stream_t stream) {
  if (M < 0 || N < 0 || workspace_bytes < 0) return QL_EINVAL;
  if (N == 0) return QL_OK;
  if (!PT || !Q || !out) return QL_EINVAL;
  if (M == 0) {  // an empty reduction: zeros (a fill kernel, not a memset node)
    hipLaunchKernelGGL(lora_wgrad_reduce, dim3(grid1d(N * kRank)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), (const float*)nullptr, 0, N,
                       out, 0.f, out_transposed != 0);
    return ql_launch_status();
  }
  if (workspace && !ql_aligned(workspace, 16)) return QL_EALIGN;
  return ql_lora_wgrad(in_dtype, PT, ldpt, Q, ldq, M, N, out, out_transposed, alpha,
                       static_cast<float*>(workspace), workspace_bytes / (int64_t)sizeof(float),
                       static_cast<hipStream_t>(stream));
}

extern "C" int qlora_lora_pack(const float* A, const float* B, int64_t K, int64_t N, float scaling,
                               int out_dtype, void* a16, void* at_pad, void* bs_pad, void* bt,
                               int pad, ql_stream_t stream) {
  if (K < 0 || N < 0 || pad < kRank || K % 8) return QL_EINVAL;
  if (K == 0 && N == 0) return QL_OK;
  if (!A || !B || !a16 || !at_pad || !bs_pad || !bt) return QL_EINVAL;
  if (out_dtype != QL_BF16 && out_dtype != QL_F16) return QL_EDTYPE;
  const int64_t total = K + N + kRank * K / 8;
  const dim3 grid(grid1d(total));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (out_dtype == QL_BF16)
    hipLaunchKernelGGL((lora_pack_kernel<QL_BF16>), grid, dim3(256), 0, s, A, B, K, N, scaling,
                       (uint16_t*)a16, (uint16_t*)at_pad, (uint16_t*)bs_pad, (uint16_t*)bt, pad);
  else
    hipLaunchKernelGGL((lora_pack_kernel<QL_F16>), grid, dim3(256), 0, s, A, B, K, N, scaling,
                       (uint16_t*)a16, (uint16_t*)at_pad, (uint16_t*)bs_pad, (uint16_t*)bt, pad);
  return ql_launch_status();
}

extern "C" int qlora_lora_pack_group(const ql_lora_factor* factors, int count, int64_t K,
                                     int out_dtype, void* a16, void* at_pad, void* bs_pad,
                                     void* bt, int pad, ql_stream_t stream) {
  if (count < 1 || count > kMaxGroup || K < 0 || K % 8 || pad < kRank * count || pad % 8)
    return QL_EINVAL;
  if (!factors || !a16 || !at_pad || !bs_pad || !bt) return QL_EINVAL;
  if (!ql_aligned(at_pad, 16) || !ql_aligned(bs_pad, 16)) return QL_EALIGN;
  if (out_dtype != QL_BF16 && out_dtype != QL_F16) return QL_EDTYPE;
  PackGroupArgs p{};
  p.G = count;
  p.off[0] = 0;
  for (int g = 0; g < count; ++g) {
    if (!factors[g].A || !factors[g].B || factors[g].n < 0) return QL_EINVAL;
    p.A[g] = factors[g].A;
    p.B[g] = factors[g].B;
    p.scale[g] = factors[g].scaling;
    p.off[g + 1] = p.off[g] + factors[g].n;
  }
  const int64_t total = K + p.off[count] + (int64_t)kRank * count * K / 8;
  if (total == 0) return QL_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (out_dtype == QL_BF16)
    hipLaunchKernelGGL((lora_pack_group_kernel<QL_BF16>), dim3(grid1d(total)), dim3(256), 0, s, p,
                       K, (uint16_t*)a16, (uint16_t*)at_pad, (uint16_t*)bs_pad, (uint16_t*)bt, pad);
  else
    hipLaunchKernelGGL((lora_pack_group_kernel<QL_F16>), dim3(grid1d(total)), dim3(256), 0, s, p,
                       K, (uint16_t*)a16, (uint16_t*)at_pad, (uint16_t*)bs_pad, (uint16_t*)bt, pad);
  return ql_launch_status();
}
