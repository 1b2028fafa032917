// Rank-16 LoRA contractions on CDNA4 matrix cores, for gfx950.
//
// The adapter GEMMs of a LoRA layer (the nn.Linear pair of solution/lora.py:172 and what
// autograd computes for it) are skinny: one side is the rank r = 16. As plain GEMMs they
// leave most of the GPU idle (a 4096 x 16 output is 32 tiles of 128 x 128). Two kernels
// cover them, both streaming the large operand from HBM exactly once, for G = 1 .. 4 adapters
// ("slots") at a time when the adapters share that operand (the q/k/v or gate/up projections
// all read the same normalised hidden state):
//
//   lora_down   out[m, c] = alpha * sum_k X[m, k] * Y[c, k]        (c < 16 G)
//               u = x A^T (forward) and du = s * g B (backward, Y = B^T): X [M, K]
//               k-contiguous, Y [16 G, K] k-contiguous (slot g in rows 16 g .. 16 g + 15).
//               Output bf16/fp16/fp32 [M, ldo] with columns 16 G .. out_cols-1 zero-filled,
//               so it can serve as the extra K = 64 segment of the base GEMM.
//   lora_wgrad  out[n, c] = alpha * sum_m Q[m, n] * P[m, c]        (c < 16 G), fp32 [N, 16 G]
//               dB = s * g^T u and dA^T = x^T du: the reduction runs over the token rows,
//               which are the strided dimension of both operands.
//
// lora_down: one workgroup (8 waves) per 16 rows and K range. A v_mfma_f32_16x16x32 needs
// 8 consecutive k per lane; the sum over k does not care which 8, so for MFMA t of a 128-k
// chunk lane l supplies k = 32 t + 8 (l/16) .. +7 of row l%16: each 16-B load instruction
// then reads 64 contiguous bytes from each of 16 rows. Y is read with the same k map, one
// fragment per slot for each fragment of X. Waves take alternate 128-k chunks and are summed
// through LDS.
//
// lora_wgrad: one workgroup (4 waves) per 128 columns and M range. Lane l loads an 8 (rows) x
// 8 (columns) block of Q as eight 16-B row pieces (lanes 0-15 of a row read 256 contiguous
// bytes), transposes it in registers with byte permutes into eight fragments that each hold
// 8 consecutive rows of one column, and multiplies them by each slot's fragment of P for the
// same 8 rows: MFMA t accumulates columns n0 + 8*(l%16) + t. Waves take alternate 32-row
// chunks and are summed through LDS.
//
// Both main loops are one straight-line block per step: every load of the step is issued
// before the first wait (a load under a branch, or a select between a load and zero inside
// the loop, splits the block and the compiler then waits for each load before the next, which
// leaves a few KiB in flight per wave and the kernel latency-bound). The load addresses are a
// wave-uniform base (scalar registers) plus a loop-invariant 32-bit lane offset. Partial
// chunks are handled after the main loop.
//
// Both kernels optionally split their reduction over blockIdx.y into an fp32 workspace,
// summed in split order by the matching reduce kernel (deterministic).
#include <mutex>
#include <type_traits>

#include "ql_philox.h"
#include "ql_swiglu.h"
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

// ---------------------------------------------------------------------------------------
constexpr int kMaxSlots = 4;    // rank-16 adapters per launch (a q/k/v or gate/up group)
constexpr int kDownWaves = 8;   // two waves per SIMD

// R: 16-row groups per lora_down workgroup. Each fragment of Y is loaded once for R fragments
// of X: a fragment of Y served from L2 costs the load path as much as one of X from HBM, and
// at R = 1 (one fragment of each) a read-pattern probe streamed X at 3.1 TB/s against 5.5
// without the Y loads (4.2 at R = 2, 4.9 at R = 4).
// U: 128-k chunks a wave keeps in flight per step.
template <int G, int R> struct DownUnroll {
  static constexpr int value = R == 1 ? (G == 1 ? 4 : 2) : 2;
};

// 16-B load from a wave-uniform base plus a per-lane 32-bit byte offset: the global load
// takes the base in scalar registers, so a stream costs one VGPR of address, not two.
QL_DEV uint4 ld16(const char* base, uint32_t off) {
  return *reinterpret_cast<const uint4*>(base + off);
}

// Lane m receives the 16 B lane src_byte / 4 holds (ds_bpermute, one per dword).
QL_DEV uint4 to_mfma_layout(const uint4& v, int src_byte) {
  return make_uint4((uint32_t)__builtin_amdgcn_ds_bpermute(src_byte, (int)v.x),
                    (uint32_t)__builtin_amdgcn_ds_bpermute(src_byte, (int)v.y),
                    (uint32_t)__builtin_amdgcn_ds_bpermute(src_byte, (int)v.z),
                    (uint32_t)__builtin_amdgcn_ds_bpermute(src_byte, (int)v.w));
}

template <int IT, int OT, bool PARTIAL, int G, int R>
__global__ __launch_bounds__(64 * kDownWaves) void lora_down_kernel(
    const uint16_t* __restrict__ X, int64_t ldx, const uint16_t* __restrict__ Y, int64_t ldy,
    int64_t M, int64_t K, int64_t k_per_split, float* __restrict__ ws,
    typename Elem<OT>::T* __restrict__ out, int64_t ldo, int out_cols, float alpha,
    uint16_t* __restrict__ out_t, int64_t ldt) {
  constexpr int U = DownUnroll<G, R>::value;
  constexpr int NC = kRank * G;
  constexpr int64_t kStride = 128 * kDownWaves;
  __shared__ f32x4_t red[R * G * kDownWaves * 64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t m0 = (int64_t)blockIdx.x * 16 * R;
  const int64_t kb = (int64_t)blockIdx.y * k_per_split;
  const int64_t ke = kb + k_per_split < K ? kb + k_per_split : K;
  // Loads use a coalesced layout (lane l: row l / 4 of a 16-row group, elements 8 (l % 4)
  // .. +7 of each 32-k group, four lanes per 64 contiguous bytes); lane permutes then move
  // each fragment to the MFMA operand layout (row l % 16, elements 8 (l / 16) .. +7).
  const int koff = 8 * (lane & 3);
  const int mfma_src = 4 * (4 * (lane & 15) + (lane >> 4));  // ds_bpermute byte address
  const char* xb = reinterpret_cast<const char*>(X + m0 * ldx);
  const char* yb = reinterpret_cast<const char*>(Y);
  uint32_t xo[R];  // row m0 + 16 r + lane / 4; rows past M read row M - 1
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = m0 + 16 * r + (lane >> 2);
    xo[r] = (uint32_t)((((row < M ? row : M - 1) - m0) * ldx + koff) * 2);
  }
  uint32_t yo[G];
#pragma unroll
  for (int g = 0; g < G; ++g) yo[g] = (uint32_t)(((16 * g + (lane >> 2)) * ldy + koff) * 2);
  f32x4_t acc[R][G][2];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int g = 0; g < G; ++g) acc[r][g][0] = acc[r][g][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Slots: wave w takes the 128-k chunks kb + 128 w + kStride j, j = 0 .. J-1. Every slot but
  // the last is whole for every wave; those are visited first, U per step, starting at slot
  // blockIdx.x mod (J - 1) so that workgroups running together read different parts of Y
  // (which every workgroup reads whole). K and the split bounds are multiples of 32, so each
  // 32-k group of the last slot is all in or all out.
  const int64_t J = (ke - kb + kStride - 1) / kStride;  // >= 1 for every launched split
  const int64_t nfull = J - 1;
  const int64_t rot = nfull > 0 ? (int64_t)blockIdx.x % nfull : 0;
  const int64_t wk = kb + 128 * wave;
  int64_t j0 = 0;
  for (; j0 + U <= nfull; j0 += U) {  // whole slots: loads only, all issued before any wait
    uint4 xv[U][R][4], yv[U][G][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int64_t js = j0 + u + rot;
      js = js >= nfull ? js - nfull : js;
      const int64_t c0 = wk + kStride * js;
      const char* xc = xb + 2 * c0;
      const char* yc = yb + 2 * c0;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int r = 0; r < R; ++r) xv[u][r][t] = ld16(xc + 64 * t, xo[r]);
#pragma unroll
        for (int g = 0; g < G; ++g) yv[u][g][t] = ld16(yc + 64 * t, yo[g]);
      }
    }
    // Keep the scheduler from interleaving the MFMAs (and register reuse) with the loads:
    // the step's loads all go out before the first wait.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int r = 0; r < R; ++r) xv[u][r][t] = to_mfma_layout(xv[u][r][t], mfma_src);
#pragma unroll
        for (int g = 0; g < G; ++g) yv[u][g][t] = to_mfma_layout(yv[u][g][t], mfma_src);
      }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int g = 0; g < G; ++g)
            acc[r][g][t & 1] = mfma<IT>(yv[u][g][t], xv[u][r][t], acc[r][g][t & 1]);
  }
  {
    // The rest (at most U slots): the remaining whole slots and the last one. A 32-k group
    // past ke, or a slot past J - 1, loads the in-range group at kb and contributes zeros; the
    // conditions are wave-uniform and the loads unconditional.
    uint4 xv[U][R][4], yv[U][G][4];
    bool ok[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = j0 + u;
      int64_t js = j + rot;
      js = js >= nfull ? js - nfull : js;
      const int64_t c0 = wk + kStride * (j < nfull ? js : nfull);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int64_t k = c0 + 32 * t;
        ok[u][t] = j < J && k < ke;
        const int64_t kk = ok[u][t] ? k : kb;
#pragma unroll
        for (int r = 0; r < R; ++r) xv[u][r][t] = ld16(xb + 2 * kk, xo[r]);
#pragma unroll
        for (int g = 0; g < G; ++g) yv[u][g][t] = ld16(yb + 2 * kk, yo[g]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int r = 0; r < R; ++r) xv[u][r][t] = to_mfma_layout(xv[u][r][t], mfma_src);
#pragma unroll
        for (int g = 0; g < G; ++g) yv[u][g][t] = to_mfma_layout(yv[u][g][t], mfma_src);
      }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int g = 0; g < G; ++g)
            acc[r][g][t & 1] = mfma<IT>(ok[u][t] ? yv[u][g][t] : z, ok[u][t] ? xv[u][r][t] : z,
                                        acc[r][g][t & 1]);
  }
  // Sum over the waves (in wave order): wave w finishes the (row group, slot) pairs w, w + 8,
  // ...; wave kDownWaves - 1 - r writes the zero columns NC .. out_cols - 1 of row group r.
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int g = 0; g < G; ++g)
      red[((r * G + g) * kDownWaves + wave) * 64 + lane] = acc[r][g][0] + acc[r][g][1];
  __syncthreads();
  const int c = 4 * (lane >> 4);  // lane holds out[row][16 g + c .. +3]
  for (int p = wave; p < R * G; p += kDownWaves) {
    const int r = p / G, g = p - (p / G) * G;
    const int64_t row = m0 + 16 * r + (lane & 15);
    if (row >= M) continue;
    f32x4_t s = red[p * kDownWaves * 64 + lane];
#pragma unroll
    for (int w = 1; w < kDownWaves; ++w) s += red[(p * kDownWaves + w) * 64 + lane];
    const int col = kRank * g + c;
    if constexpr (PARTIAL) {
      *reinterpret_cast<float4*>(ws + ((int64_t)blockIdx.y * M + row) * NC + col) =
          make_float4(s[0], s[1], s[2], s[3]);
    } else {
      auto* o = out + row * ldo;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[col + e] = Elem<OT>::from_f32(alpha * s[e]);
      if (out_t) {  // [NC, M]: the 16 lanes of a row group write 32 contiguous bytes per column
#pragma unroll
        for (int e = 0; e < 4; ++e)
          out_t[(int64_t)(col + e) * ldt + row] = Elem<IT>::from_f32(alpha * s[e]);
      }
    }
  }
  if constexpr (!PARTIAL) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = m0 + 16 * r + (lane & 15);
      if (wave != kDownWaves - 1 - r || row >= M) continue;
      auto* o = out + row * ldo;
      for (int zc = NC + c; zc < out_cols; zc += 16)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (zc + e < out_cols) o[zc + e] = Elem<OT>::from_f32(0.f);
    }
  }
}

// alpha scales columns 0 .. 15 and alpha_hi the rest (the two adapters of the fused SwiGLU
// backward have their own scalings; lora_down passes the same value twice).
template <int IT, int OT>
__global__ __launch_bounds__(256) void lora_down_reduce(const float* __restrict__ ws, int splits,
                                                        int64_t M, int nc,
                                                        typename Elem<OT>::T* __restrict__ out,
                                                        int64_t ldo, int out_cols, float alpha,
                                                        float alpha_hi,
                                                        uint16_t* __restrict__ out_t, int64_t ldt) {
  const int64_t total = M * out_cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / out_cols;
    const int c = (int)(i - m * out_cols);
    float v = 0.f;
    if (c < nc) {
      // 8 partials loaded at a time, added in split order
      const float* wp = ws + m * nc + c;
      const int64_t stride = M * nc;
      int z = 0;
      for (; z + 8 <= splits; z += 8) {
        float w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = wp[(int64_t)(z + j) * stride];
#pragma unroll
        for (int j = 0; j < 8; ++j) v += w[j];
      }
      for (; z < splits; ++z) v += wp[(int64_t)z * stride];
      v *= c < kRank ? alpha : alpha_hi;
      if (out_t) out_t[(int64_t)c * ldt + m] = Elem<IT>::from_f32(v);
    }
    out[m * ldo + c] = Elem<OT>::from_f32(v);
  }
}

// ---------------------------------------------------------------------------------------
// SwiGLU backward fused with the down-projections of its two gradients (the gate and up
// adapters' du of a LoRA MLP):
//   dgate, dup     = the SwiGLU gradients of (grad, gate, up)     stored, as swiglu_bwd_rows
//   out[m, c]      = alpha_g * sum_k dgate[m, k] * YG[c, k]        c < 16
//   out[m, 16 + c] = alpha_u * sum_k dup[m, k] * YU[c, k]
// A streaming kernel: a workgroup of 4 waves takes 32 rows and a K range and walks it in
// tiles of 32 x 256. Thread t loads, for rows t / 32 + 8 h (h = 0 .. 3), the 16 B at k = 8
// (t % 32) of grad, gate and up (each load instruction reads two whole 512-B row pieces),
// computes both gradients, stores them (nontemporal: they are not read again here and are
// larger than the caches) and also writes them to an LDS copy of the tile. After one barrier
// wave w reads the 16 x 32 fragments of k groups 2w and 2w + 1 of both row groups from LDS
// in the MFMA operand layout (row l % 16, k = 32 g + 8 (l / 16) .. +7) and multiplies them
// by the matching fragments of YG and YU (from L2; each serves both row groups). The LDS
// tile is double buffered, so the barrier of the next tile also orders this tile's reads
// before their buffer is written again; rows are padded by 16 B so the 16 rows of a fragment
// read fall in different banks. Each tile tests its gate values once and runs one of two
// copies of the arithmetic: the sigmoid's fast reciprocal or the division (ql_swiglu.h).
//
// Measured on MI355X at 4096 x 18944 bf16 (775.9 MB per call): 161 us, 4.8 TB/s, against
// 207 us for a kernel that loaded 16 rows x 64 B per instruction and multiplied straight from
// registers (one 8-wave workgroup per CU, each wave alternating a 32 KB load burst with its
// arithmetic); the plain qlora_swiglu_bwd_rows takes 150 us. Wider tiles (512 or 1024 k:
// fewer, longer row pieces), 16-row tiles and a software-pipelined variant (the next tile's
// loads issued before this tile's arithmetic) all measured 1-15% slower; the per-tile test
// costs 3 us against the fast reciprocal without it.
// LoRA dropout on h = silu(gate) up, the input of the down projection's adapter (its own seed):
// the forward draws keep and stores it as bits, and its u products take the dropped values; the
// backward's recomputed h for that adapter's lora_A gradient is dropped with the same bits.
struct SwDrop {
  uint64_t seed;
  uint32_t thr;     // ql_philox::keep_threshold(p)
  float scale;      // 1 / (1 - p)
  uint8_t* bits;    // 8 x 8 blocks (ql_philox.h)
  int64_t gs;       // their group stride
  // backward only: the down adapter's masked rank-16 term added to the incoming gradient,
  // grad + scale * keep (du[:, :16] a) (a [16, K]); du null: none
  const uint16_t* add_du;
  int64_t add_ldu;
  const uint16_t* add_a;
  int64_t add_lda;
};

// v_mfma_f32_16x16x16 (one rank-16 product per output), the instruction of the masked adds in
// lora.hip: D[i][j] = sum_r a[i][r] b[r][j], lane l supplying a[l % 16][4 (l / 16) .. +3] and
// b[4 (l / 16) .. +3][l % 16] and holding D[4 (l / 16) + e][l % 16] in element e.
template <int DT> QL_DEV f32x4_t mfma_k16(const uint2& a, const uint2& b);
template <> QL_DEV f32x4_t mfma_k16<QL_BF16>(const uint2& a, const uint2& b) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(v4i16, a),
                                                  __builtin_bit_cast(v4i16, b),
                                                  f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
}
template <> QL_DEV f32x4_t mfma_k16<QL_F16>(const uint2& a, const uint2& b) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, a), __builtin_bit_cast(h4, b),
                                              f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
}

constexpr int kSwRows = 32;                 // rows per workgroup (two 16-row MFMA groups)
constexpr int kSwK = 256;                   // k per tile
constexpr int kSwLdsRow = 2 * kSwK + 16;    // bytes per LDS row
constexpr int kSwLdsArr = kSwRows * kSwLdsRow;  // one gradient's tile
constexpr int kSwLdsBuf = 2 * kSwLdsArr;    // dgate + dup

template <int IT, bool PARTIAL>
__global__ __launch_bounds__(256) void swiglu_bwd_down_kernel(
    const uint16_t* __restrict__ GR, int64_t ldgr, const uint16_t* __restrict__ GA,
    int64_t ldga, const uint16_t* __restrict__ UP, int64_t ldup, uint16_t* __restrict__ DG,
    int64_t lddg, uint16_t* __restrict__ DU, int64_t lddu, const uint16_t* __restrict__ YG,
    const uint16_t* __restrict__ YU, int64_t ldy, int64_t M, int64_t K, int64_t k_per_split,
    float* __restrict__ ws, uint16_t* __restrict__ out, int64_t ldo, int out_cols,
    float alpha_g, float alpha_u, uint16_t* __restrict__ out_t, int64_t ldt) {
  constexpr int NC = 2 * kRank;
  constexpr int RG = kSwRows / 16;  // 16-row MFMA groups
  constexpr int H = kSwRows / 8;    // rows per thread
  typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
  static_assert(2 * kSwLdsBuf >= RG * 2 * 4 * 64 * 16, "the wave reduction reuses the tiles");
  __shared__ __attribute__((aligned(16))) char lds[2 * kSwLdsBuf];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t m0 = (int64_t)blockIdx.x * kSwRows;
  const int64_t kb = (int64_t)blockIdx.y * k_per_split;
  const int64_t ke = kb + k_per_split < K ? kb + k_per_split : K;
  const int lr = tid >> 5, c = tid & 31;
  // wave-uniform bases at row m0; lane offsets of rows m0 + lr + 8 h (a row past M works on
  // row M - 1 and stores the bits row M - 1's owner stores)
  const char* grb = reinterpret_cast<const char*>(GR + m0 * ldgr);
  const char* gab = reinterpret_cast<const char*>(GA + m0 * ldga);
  const char* upb = reinterpret_cast<const char*>(UP + m0 * ldup);
  char* dgb = reinterpret_cast<char*>(DG + m0 * lddg);
  char* dub = reinterpret_cast<char*>(DU + m0 * lddu);
  uint32_t ogr[H], oga[H], oup[H], odg[H], odu[H];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    const int64_t row = m0 + lr + 8 * h;
    const int64_t rs = (row < M ? row : M - 1) - m0;
    ogr[h] = (uint32_t)(rs * ldgr * 2);
    oga[h] = (uint32_t)(rs * ldga * 2);
    oup[h] = (uint32_t)(rs * ldup * 2);
    odg[h] = (uint32_t)(rs * lddg * 2);
    odu[h] = (uint32_t)(rs * lddu * 2);
  }
  const uint32_t oy = (uint32_t)(((lane & 15) * ldy + 8 * (lane >> 4)) * 2);
  const int lds_w = lr * kSwLdsRow + 16 * c;                       // + 8 h rows
  const int lds_r = (lane & 15) * kSwLdsRow + 16 * (lane >> 4);   // + 16 rg rows + 64 g
  f32x4_t acc[RG][2][2];  // [row group][gate / up][k group parity]
#pragma unroll
  for (int rg = 0; rg < RG; ++rg)
#pragma unroll
    for (int q = 0; q < 2; ++q) acc[rg][q][0] = acc[rg][q][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  int buf = 0;
  for (int64_t k0 = kb; k0 < ke; k0 += kSwK) {
    // In the last tile of the range, chunks and 32-k groups past ke read the chunk / group
    // at k0: recomputed and stored with the same bits, and left out of the products.
    const int64_t kx = k0 + 8 * c < ke ? k0 + 8 * c : k0;
    const uint32_t kxb = (uint32_t)(2 * kx);
    uint4 vgr[H], vga[H], vup[H], yv[2][2];
    // the gate values first: the test below needs all of them, the rows only their own
#pragma unroll
    for (int h = 0; h < H; ++h) vga[h] = ld16(gab, oga[h] + kxb);
#pragma unroll
    for (int h = 0; h < H; ++h) {
      vgr[h] = ld16(grb, ogr[h] + kxb);
      vup[h] = ld16(upb, oup[h] + kxb);
    }
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const int64_t kg = k0 + 32 * (2 * wave + gi);
      const int64_t ky = kg < ke ? kg : k0;
      yv[0][gi] = ld16(reinterpret_cast<const char*>(YG) + 2 * ky, oy);
      yv[1][gi] = ld16(reinterpret_cast<const char*>(YU) + 2 * ky, oy);
    }
    char* lb = lds + buf * kSwLdsBuf;
    // one test of the tile's gate values picks the sigmoid's reciprocal for all of them
    bool fast = true;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      float ga8[8];
      Vec8<IT>::unpack(vga[h], ga8);
      fast &= ql_sigmoid_fast_ok8(ga8);
    }
    auto rows = [&](auto fast_tag) {
#pragma unroll
      for (int h = 0; h < H; ++h) {
        float gr8[8], ga8[8], up8[8], dg8[8], du8[8];
        Vec8<IT>::unpack(vgr[h], gr8);
        Vec8<IT>::unpack(vga[h], ga8);
        Vec8<IT>::unpack(vup[h], up8);
        ql_swiglu_bwd8_as<decltype(fast_tag)::value>(gr8, ga8, up8, dg8, du8);
        const uint4 pdg = Vec8<IT>::pack(dg8);
        const uint4 pdu = Vec8<IT>::pack(du8);
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4v, pdg),
                                    reinterpret_cast<u32x4v*>(dgb + odg[h] + kxb));
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4v, pdu),
                                    reinterpret_cast<u32x4v*>(dub + odu[h] + kxb));
        *reinterpret_cast<uint4*>(lb + lds_w + 8 * h * kSwLdsRow) = pdg;
        *reinterpret_cast<uint4*>(lb + kSwLdsArr + lds_w + 8 * h * kSwLdsRow) = pdu;
      }
    };
    if (__builtin_expect(fast, 1)) rows(std::true_type{});
    else rows(std::false_type{});
    __syncthreads();
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        const int off = lds_r + 16 * rg * kSwLdsRow + 64 * (2 * wave + gi);
        const uint4 fdg = *reinterpret_cast<const uint4*>(lb + off);
        const uint4 fdu = *reinterpret_cast<const uint4*>(lb + kSwLdsArr + off);
        if (k0 + 32 * (2 * wave + gi) < ke) {  // wave-uniform
          acc[rg][0][gi] = mfma<IT>(yv[0][gi], fdg, acc[rg][0][gi]);
          acc[rg][1][gi] = mfma<IT>(yv[1][gi], fdu, acc[rg][1][gi]);
        }
      }
    }
    buf ^= 1;
  }
  // Sum over the waves in wave order through LDS (after a barrier: the last tile's reads are
  // done); wave p < 2 RG then finishes row group p / 2, adapter p % 2.
  __syncthreads();
  f32x4_t* red = reinterpret_cast<f32x4_t*>(lds);
#pragma unroll
  for (int rg = 0; rg < RG; ++rg)
#pragma unroll
    for (int q = 0; q < 2; ++q)
      red[((rg * 2 + q) * 4 + wave) * 64 + lane] = acc[rg][q][0] + acc[rg][q][1];
  __syncthreads();
  const int cc = 4 * (lane >> 4);
  if (wave < 2 * RG) {
    const int rg = wave >> 1, q = wave & 1;
    const int64_t row = m0 + 16 * rg + (lane & 15);
    if (row < M) {
      f32x4_t sum = red[(wave * 4) * 64 + lane];
#pragma unroll
      for (int w = 1; w < 4; ++w) sum += red[(wave * 4 + w) * 64 + lane];
      const int col = kRank * q + cc;
      if constexpr (PARTIAL) {
        *reinterpret_cast<float4*>(ws + ((int64_t)blockIdx.y * M + row) * NC + col) =
            make_float4(sum[0], sum[1], sum[2], sum[3]);
      } else {
        const float a = q ? alpha_u : alpha_g;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint16_t v = Elem<IT>::from_f32(a * sum[e]);
          out[row * ldo + col + e] = v;
          if (out_t) out_t[(int64_t)(col + e) * ldt + row] = v;
        }
      }
    }
  }
  if constexpr (!PARTIAL) {
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {  // wave 3 - rg writes the zero columns of row group rg
      const int64_t row = m0 + 16 * rg + (lane & 15);
      if (wave != 3 - rg || row >= M) continue;
      for (int zc = NC + cc; zc < out_cols; zc += 16)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (zc + e < out_cols) out[row * ldo + zc + e] = Elem<IT>::from_f32(0.f);
    }
  }
}

// ---------------------------------------------------------------------------------------
// SwiGLU backward fused with both rank-16 products of its gradients for the gate and up
// adapters (a LoRA MLP): for d in {dgate, dup} with that adapter's Y [16, K] and u^T [16, M],
//   du[m, c] (16 columns each)  = alpha * sum_k d[m, k] Y[c, k]    the down-projection
//   dB[k, c]                    = beta  * sum_m d[m, k] u[m, c]    the lora_B gradient
// A workgroup owns 256 columns and a range of rows (a multiple of 32) and walks it in tiles
// of 32 x 256, loading, computing and storing exactly as swiglu_bwd_down_kernel does (the
// same ql_swiglu.h arithmetic, the same bits) and keeping both gradients of the tile in LDS.
// After the tile's barrier:
//  - du: wave w takes row group w / 2 and adapter w % 2: its 8 products over the 256 columns
//    use that adapter's Y fragments, loaded once per workgroup (the columns are fixed), and
//    the fp32 partial of the 16 x 16 block goes to ws_du[column block][row][32]; the partials
//    of the column blocks are summed in order by lora_down_reduce.
//  - dB: wave w takes 16-column blocks 4w .. 4w + 3 of both adapters; each product reads the
//    block transposed from LDS (two ds_read_b64_tr_b16: 8 consecutive rows of one column per
//    lane) against u^T's 32 rows of the tile (rows past M read as zero), accumulating over the
//    workgroup's rows; at the end the partial goes to ws_db[adapter][row range][K][16], summed
//    in order by lora_wgrad_reduce.
// So the gradients are never read back from HBM for either product; the extra traffic is the
// fp32 partials (M x 32 per column block, K x 32 per row range).
// DA: also the lora_A gradient of the next layer's adapter, whose input was h = silu(gate) up:
//   dA^T[k, c] = sum_m h[m, k] ud[m, c]   (ud = that adapter's du, given as ud^T [16, M])
// with h recomputed in registers (the bits of the forward) into a third LDS array and read
// transposed like the gradients. The three arrays take one LDS buffer (with a second barrier
// per tile before it is refilled) and the Y fragments move from registers to LDS, so two
// workgroups (at most 256 registers a lane) still fit on a CU.
// DROP with dr.add_du: the incoming gradient first gets the down adapter's term through its
// dropout mask, grad + scale * keep (du a), rounded to the input type: the sum
// qlora_lora_up_masked_add writes, from the same products (one v_mfma_f32_16x16x16 per 16 x 16
// block, C = 0, the a fragments staged in LDS once per workgroup) and the same fp32 steps, so
// the gradients are those of the separate add followed by this kernel, bit for bit. The
// products of a tile go through the (not yet written) gradient arrays of the LDS buffer,
// with two more barriers a tile.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

// Transposing LDS read (ds_read_b64_tr_b16): within each 16-lane group, with lane 4 j + c
// addressing row r_j, columns n0 + 4 c .. +3 of a row-major 16-bit tile, lane i receives
// column n0 + i of rows r_0 .. r_3.
QL_DEV uint2 lds_read_tr(const char* p) {
  const v4i16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(p));
  return __builtin_bit_cast(uint2, r);
}

constexpr int kSlRows = 32;                          // rows per tile
constexpr int kSlCols = 256;                         // columns per workgroup
constexpr int kSlLdsRow = 2 * kSlCols + 16;          // bytes per LDS row (16 B of padding)
constexpr int kSlLdsArr = kSlRows * kSlLdsRow;       // one gradient's tile
constexpr int kSlLdsBuf = 2 * kSlLdsArr;             // dgate + dup

template <int IT, bool DA, bool DROP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void swiglu_bwd_lora_kernel(
    const uint16_t* __restrict__ GR, int64_t ldgr, const uint16_t* __restrict__ GA,
    int64_t ldga, const uint16_t* __restrict__ UP, int64_t ldup, uint16_t* __restrict__ DG,
    int64_t lddg, uint16_t* __restrict__ DU, int64_t lddu, const uint16_t* __restrict__ YG,
    const uint16_t* __restrict__ YU, int64_t ldy, const uint16_t* __restrict__ UTG,
    const uint16_t* __restrict__ UTU, int64_t ldut, int64_t M, int64_t K,
    int64_t rows_per_split, float* __restrict__ ws_du, float* __restrict__ ws_db,
    const uint16_t* __restrict__ UTD, float* __restrict__ ws_da, SwDrop dr) {
  static_assert(DA || !DROP, "the mask applies to the recomputed h of the lora_A gradient");
  typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
  constexpr int NA = DA ? 3 : 2;          // LDS arrays per tile: dgate, dup (, h)
  constexpr int NBUF = DA ? 1 : 2;        // tiles in LDS
  constexpr int BUF = NA * kSlLdsArr;
  // DA: the Y fragments live in LDS (16 rows of 256 columns per adapter, rows padded like the
  // tiles), not in registers, which keeps the kernel at two waves per SIMD
  constexpr int YBYTES = DA ? 2 * 16 * kSlLdsRow : 0;
  // DROP: the a fragments of the fused masked add, [16-column block][lane], 8 B each
  constexpr int AFBYTES = DROP ? (kSlCols / 16) * 64 * 8 : 0;
  constexpr int kTermRow = 4 * kSlCols + 16;  // bytes per row of a tile's fp32 products
  static_assert(!DROP || kSlRows * kTermRow <= 2 * kSlLdsArr, "products fit the gradient arrays");
  __shared__ __attribute__((aligned(16))) char lds[NBUF * BUF + YBYTES + AFBYTES];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t k0 = (int64_t)blockIdx.x * kSlCols;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_split;
  const int64_t r1 = r0 + rows_per_split < M ? r0 + rows_per_split : M;
  const int lr = tid >> 5, c = tid & 31;
  // this thread's 16-B chunk: columns past K (the last block) recompute the block's first
  const int64_t kx = k0 + 8 * c < K ? k0 + 8 * c : k0;
  const int rg = wave >> 1, qd = wave & 1;  // du: row group and adapter of this wave
  uint4 yv[DA ? 1 : kSlCols / 32];
  char* const ylds = lds + NBUF * BUF;
  if constexpr (DA) {  // thread t: rows t / 32 and t / 32 + 8 of both Y, 16 B at column 8 (t % 32)
    const int64_t col = k0 + 8 * c < K ? k0 + 8 * c : k0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = lr + 8 * i;
#pragma unroll
      for (int a = 0; a < 2; ++a)
        *reinterpret_cast<uint4*>(ylds + (a * 16 + r) * kSlLdsRow + 16 * c) =
            *reinterpret_cast<const uint4*>((a ? YU : YG) + (int64_t)r * ldy + col);
    }
  } else {
    const uint16_t* yq = qd ? YU : YG;
    const uint32_t oy = (uint32_t)(((lane & 15) * ldy + 8 * (lane >> 4)) * 2);
#pragma unroll
    for (int g = 0; g < kSlCols / 32; ++g) {
      const int64_t kg = k0 + 32 * g;
      yv[g] = ld16(reinterpret_cast<const char*>(yq + (kg < K ? kg : k0)), oy);
    }
  }
  char* const aflds = lds + NBUF * BUF + YBYTES;
  const bool madd = DROP && dr.add_du != nullptr;  // uniform
  if constexpr (DROP) {
    if (madd) {  // lane (r, q) of block t: a[4 q + e][k0 + 16 t + r], e = 0 .. 3 (zero past K)
#pragma unroll
      for (int j = 0; j < (kSlCols / 16) * 64 / 256; ++j) {
        const int e8 = tid + 256 * j;
        const int t = e8 >> 6, l = e8 & 63;
        const int64_t col = k0 + 16 * t + (l & 15);
        uint16_t hv[4] = {0, 0, 0, 0};
        if (col < K) {
#pragma unroll
          for (int e = 0; e < 4; ++e) hv[e] = dr.add_a[(int64_t)(4 * (l >> 4) + e) * dr.add_lda + col];
        }
        *reinterpret_cast<uint2*>(aflds + 8 * e8) =
            make_uint2(hv[0] | (uint32_t)hv[1] << 16, hv[2] | (uint32_t)hv[3] << 16);
      }
      __syncthreads();
    }
  }
  f32x4_t acc_db[4][NA];  // [column block 4 wave + i][adapter (, dA)]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int q = 0; q < NA; ++q) acc_db[i][q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int lds_w = lr * kSlLdsRow + 16 * c;                            // + 8 h rows
  const int lds_r = (lane & 15) * kSlLdsRow + 16 * (lane >> 4);         // + 16 rg rows + 64 g
  const int lds_t = (8 * (lane >> 4) + ((lane >> 2) & 3)) * kSlLdsRow + 8 * (lane & 3);
  int buf = 0;
  // DROP with the masked add: lane's row 16 rg + lane % 16 of the tile at row m, columns
  // 4 (lane / 16) .. +3 of du (the second operand of the products)
  auto load_dv = [&](int64_t m) {
    const int64_t rd = m + 16 * rg + (lane & 15) < M ? m + 16 * rg + (lane & 15) : M - 1;
    return *reinterpret_cast<const uint2*>(dr.add_du + rd * dr.add_ldu + 4 * (lane >> 4));
  };
  uint2 dv_next = make_uint2(0, 0);
  if constexpr (DROP) {
    if (madd && r0 < r1) dv_next = load_dv(r0);
  }
  for (int64_t m0 = r0; m0 < r1; m0 += kSlRows) {
    // rows m0 + lr + 8 h; a row past M (the last tile) works on row M - 1 and stores the
    // bits row M - 1's owner stores, and is left out of both products
    uint32_t ogr[4], oga[4], oup[4];
    auto row_of = [&](int h) { return m0 + lr + 8 * h < M ? lr + 8 * h : (int)(M - 1 - m0); };
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int64_t rs = row_of(h);
      ogr[h] = (uint32_t)((rs * ldgr + kx) * 2);
      oga[h] = (uint32_t)((rs * ldga + kx) * 2);
      oup[h] = (uint32_t)((rs * ldup + kx) * 2);
    }
    const char* grb = reinterpret_cast<const char*>(GR + m0 * ldgr);
    const char* gab = reinterpret_cast<const char*>(GA + m0 * ldga);
    const char* upb = reinterpret_cast<const char*>(UP + m0 * ldup);
    char* dgb = reinterpret_cast<char*>(DG + m0 * lddg);
    char* dub = reinterpret_cast<char*>(DU + m0 * lddu);
    uint4 vgr[4], vga[4], vup[4], uq[NA];
    uint32_t kbyte[4];  // DROP: the keep byte of each of this thread's rows at columns kx ..
    const uint2 dv = dv_next;  // the masked add's du operand, loaded a tile ahead
    if constexpr (DROP) {
      if (madd && m0 + kSlRows < r1) dv_next = load_dv(m0 + kSlRows);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int64_t rowc = m0 + lr + 8 * h < M ? m0 + lr + 8 * h : M - 1;
        kbyte[h] = dr.bits[ql_philox::keep_byte(rowc, kx, dr.gs)];
      }
    }
#pragma unroll
    for (int h = 0; h < 4; ++h) vga[h] = ld16(gab, oga[h]);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      vgr[h] = ld16(grb, ogr[h]);
      vup[h] = ld16(upb, oup[h]);
    }
    // dB's (and dA's) second operand: u^T row lane % 16, tile rows 8 (lane / 16) .. +7
    const int64_t ur = m0 + 8 * (lane >> 4);
#pragma unroll
    for (int q = 0; q < NA; ++q) {
      const uint16_t* ut = (q == 2 ? UTD : q ? UTU : UTG) + (int64_t)(lane & 15) * ldut;
      if (ur + 8 <= M) {
        uq[q] = *reinterpret_cast<const uint4*>(ut + ur);
      } else {
        uint16_t v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = ur + i < M ? ut[ur + i] : (uint16_t)0;
        uq[q] = make_uint4((uint32_t)v[0] | ((uint32_t)v[1] << 16),
                           (uint32_t)v[2] | ((uint32_t)v[3] << 16),
                           (uint32_t)v[4] | ((uint32_t)v[5] << 16),
                           (uint32_t)v[6] | ((uint32_t)v[7] << 16));
      }
    }
    char* lb = lds + buf * BUF;
    if (NBUF == 1 && m0 != r0) __syncthreads();  // the previous tile's reads are done
    if constexpr (DROP) {
      if (madd) {
        // wave w: rows 16 rg .. +15, column blocks 8 qd .. +7 of the tile's products
#pragma unroll
        for (int tt = 0; tt < kSlCols / 32; ++tt) {
          const int t = (kSlCols / 32) * qd + tt;
          const uint2 af = *reinterpret_cast<const uint2*>(aflds + 8 * (t * 64 + lane));
          const f32x4_t pr = mfma_k16<IT>(af, dv);
          *reinterpret_cast<f32x4_t*>(lb + (16 * rg + (lane & 15)) * kTermRow +
                                      4 * (16 * t + 4 * (lane >> 4))) = pr;
        }
        __syncthreads();
        {
#pragma clang fp contract(off)  // scale * kept, then the add: two roundings, as the masked add
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const float* tp =
              reinterpret_cast<const float*>(lb + row_of(h) * kTermRow + 4 * (kx - k0));
          const f32x4_t p0 = *reinterpret_cast<const f32x4_t*>(tp);
          const f32x4_t p1 = *reinterpret_cast<const f32x4_t*>(tp + 4);
          const float pv[8] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
          float v[8];
          Vec8<IT>::unpack(vgr[h], v);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float kept = -0.0f + ((kbyte[h] >> e) & 1u ? pv[e] : -0.0f);
            v[e] = v[e] + dr.scale * kept;
          }
          vgr[h] = Vec8<IT>::pack(v);
        }
        }
        __syncthreads();  // every product is read before the gradients overwrite them
      }
    }
    bool fast = true;  // one test of the tile's gate values (ql_swiglu.h)
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      float ga8[8];
      Vec8<IT>::unpack(vga[h], ga8);
      fast &= ql_sigmoid_fast_ok8(ga8);
    }
    auto rows = [&](auto fast_tag) {
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        float gr8[8], ga8[8], up8[8], dg8[8], du8[8];
        Vec8<IT>::unpack(vgr[h], gr8);
        Vec8<IT>::unpack(vga[h], ga8);
        Vec8<IT>::unpack(vup[h], up8);
        ql_swiglu_bwd8_as<decltype(fast_tag)::value>(gr8, ga8, up8, dg8, du8);
        const uint4 pdg = Vec8<IT>::pack(dg8);
        const uint4 pdu = Vec8<IT>::pack(du8);
        // the store offsets are formed here, not kept from the loads (registers)
        const uint32_t rsu = (uint32_t)row_of(h), kxu = (uint32_t)kx;
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4v, pdg),
                                    reinterpret_cast<u32x4v*>(dgb + 2u * (rsu * (uint32_t)lddg + kxu)));
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4v, pdu),
                                    reinterpret_cast<u32x4v*>(dub + 2u * (rsu * (uint32_t)lddu + kxu)));
        *reinterpret_cast<uint4*>(lb + lds_w + 8 * h * kSlLdsRow) = pdg;
        *reinterpret_cast<uint4*>(lb + kSlLdsArr + lds_w + 8 * h * kSlLdsRow) = pdu;
        if constexpr (DA) {
          float h8[8];
          ql_swiglu_fwd8_as<decltype(fast_tag)::value>(ga8, up8, h8);
          uint4 ph = Vec8<IT>::pack(h8);
          if constexpr (DROP) {  // the forward's dropped value of h, from its keep bits
            float hv[8];
            Vec8<IT>::unpack(ph, hv);
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = (kbyte[h] >> e) & 1u ? hv[e] * dr.scale : 0.0f;
            ph = Vec8<IT>::pack(hv);
          }
          *reinterpret_cast<uint4*>(lb + 2 * kSlLdsArr + lds_w + 8 * h * kSlLdsRow) = ph;
        }
      }
    };
    if (__builtin_expect(fast, 1)) rows(std::true_type{});
    else rows(std::false_type{});
    // this tile's LDS copy is complete; with two buffers, every wave has also finished
    // reading the copy two tiles back, which the next tile overwrites
    __syncthreads();
    {
      f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < kSlCols / 32; ++g) {
        const uint4 f = *reinterpret_cast<const uint4*>(lb + qd * kSlLdsArr + lds_r +
                                                        16 * rg * kSlLdsRow + 64 * g);
        uint4 y;
        if constexpr (DA)
          y = *reinterpret_cast<const uint4*>(ylds + (qd * 16 + (lane & 15)) * kSlLdsRow +
                                              64 * g + 16 * (lane >> 4));
        else
          y = yv[g];
        if (k0 + 32 * g < K) acc = mfma<IT>(y, f, acc);  // wave-uniform
      }
      const int64_t row = m0 + 16 * rg + (lane & 15);
      if (row < M)
        *reinterpret_cast<float4*>(ws_du + ((int64_t)blockIdx.x * M + row) * (2 * kRank) +
                                   kRank * qd + 4 * (lane >> 4)) =
            make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n0 = 16 * (4 * wave + i);
      if (k0 + n0 < K) {  // wave-uniform; K % 32 == 0: a 16-column block is all in or out
#pragma unroll
        for (int q = 0; q < NA; ++q) {
          const char* p = lb + q * kSlLdsArr + lds_t + 2 * n0;
          const uint2 a = lds_read_tr(p);                   // rows 8 (lane / 16) + 0 .. 3
          const uint2 b = lds_read_tr(p + 4 * kSlLdsRow);   // rows 8 (lane / 16) + 4 .. 7
          acc_db[i][q] = mfma<IT>(make_uint4(a.x, a.y, b.x, b.y), uq[q], acc_db[i][q]);
        }
      }
    }
    if (NBUF == 2) buf ^= 1;
  }
  // lane holds dB[n = block + 4 (lane / 16) + e][c = lane % 16]
  const int S = (int)gridDim.y;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t n0 = k0 + 16 * (4 * wave + i);
    if (n0 >= K) continue;
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        ws_db[(((int64_t)q * S + blockIdx.y) * K + n0 + 4 * (lane >> 4) + e) * kRank +
              (lane & 15)] = acc_db[i][q][e];
    if constexpr (DA) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        ws_da[((int64_t)blockIdx.y * K + n0 + 4 * (lane >> 4) + e) * kRank + (lane & 15)] =
            acc_db[i][2][e];
    }
  }
}

// ---------------------------------------------------------------------------------------
// SwiGLU forward fused with the down-projection of its output by the next layer's adapter
// (the down projection of a LoRA MLP):
//   h        = silu(gate) * up             stored, the bits of qlora_swiglu_fwd_rows
//   out[m, c] = alpha * sum_k h[m, k] Y[c, k]   c < 16 (Y = that adapter's A [16, K])
// The same streaming tile walk as swiglu_bwd_down_kernel (32 x 256 tiles of a row block over
// a K range, one LDS copy of each tile, one barrier per tile), with two inputs, one output and
// one product: wave w multiplies k groups 2w and 2w + 1 of both row groups by Y's fragments
// (from L2, each serving both row groups), and the waves' sums meet in LDS at the end.
template <int IT, bool PARTIAL, bool DROP>
__global__ __launch_bounds__(256) void swiglu_fwd_down_kernel(
    const uint16_t* __restrict__ GA, int64_t ldga, const uint16_t* __restrict__ UP,
    int64_t ldup, uint16_t* __restrict__ HH, int64_t ldh, const uint16_t* __restrict__ Y,
    int64_t ldy, int64_t M, int64_t K, int64_t k_per_split, float* __restrict__ ws,
    uint16_t* __restrict__ out, int64_t ldo, int out_cols, float alpha,
    uint16_t* __restrict__ out_t, int64_t ldt, SwDrop dr) {
  constexpr int RG = kSwRows / 16;
  constexpr int H = kSwRows / 8;
  typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
  static_assert(kSwLdsBuf >= RG * 4 * 64 * 16, "the wave reduction reuses the tiles");
  __shared__ __attribute__((aligned(16))) char lds[2 * kSwLdsArr];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t m0 = (int64_t)blockIdx.x * kSwRows;
  const int64_t kb = (int64_t)blockIdx.y * k_per_split;
  const int64_t ke = kb + k_per_split < K ? kb + k_per_split : K;
  const int lr = tid >> 5, c = tid & 31;
  // rows m0 + lr + 8 h; a row past M works on row M - 1 and stores the bits its owner stores
  const char* gab = reinterpret_cast<const char*>(GA + m0 * ldga);
  const char* upb = reinterpret_cast<const char*>(UP + m0 * ldup);
  char* hb = reinterpret_cast<char*>(HH + m0 * ldh);
  uint32_t oga[H], oup[H], oh[H];
  int64_t rowc[H];  // the row each of this thread's rows works on (row M - 1 past M)
#pragma unroll
  for (int h = 0; h < H; ++h) {
    const int64_t row = m0 + lr + 8 * h;
    const int64_t rs = (row < M ? row : M - 1) - m0;
    rowc[h] = m0 + rs;
    oga[h] = (uint32_t)(rs * ldga * 2);
    oup[h] = (uint32_t)(rs * ldup * 2);
    oh[h] = (uint32_t)(rs * ldh * 2);
  }
  const uint32_t oy = (uint32_t)(((lane & 15) * ldy + 8 * (lane >> 4)) * 2);
  const int lds_w = lr * kSwLdsRow + 16 * c;
  const int lds_r = (lane & 15) * kSwLdsRow + 16 * (lane >> 4);
  f32x4_t acc[RG][2];  // [row group][k group parity]
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) acc[rg][0] = acc[rg][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  int buf = 0;
  for (int64_t k0 = kb; k0 < ke; k0 += kSwK) {
    // chunks and 32-k groups past ke read the chunk / group at k0: recomputed and stored with
    // the same bits, and left out of the products
    const int64_t kx = k0 + 8 * c < ke ? k0 + 8 * c : k0;
    const uint32_t kxb = (uint32_t)(2 * kx);
    uint4 vga[H], vup[H], yv[2];
#pragma unroll
    for (int h = 0; h < H; ++h) vga[h] = ld16(gab, oga[h] + kxb);
#pragma unroll
    for (int h = 0; h < H; ++h) vup[h] = ld16(upb, oup[h] + kxb);
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const int64_t kg = k0 + 32 * (2 * wave + gi);
      yv[gi] = ld16(reinterpret_cast<const char*>(Y) + 2 * (kg < ke ? kg : k0), oy);
    }
    char* lb = lds + buf * kSwLdsArr;
    bool fast = true;  // one test of the tile's gate values (ql_swiglu.h)
#pragma unroll
    for (int h = 0; h < H; ++h) {
      float ga8[8];
      Vec8<IT>::unpack(vga[h], ga8);
      fast &= ql_sigmoid_fast_ok8(ga8);
    }
    auto rows = [&](auto fast_tag) {
#pragma unroll
      for (int h = 0; h < H; ++h) {
        float ga8[8], up8[8], h8[8];
        Vec8<IT>::unpack(vga[h], ga8);
        Vec8<IT>::unpack(vup[h], up8);
        ql_swiglu_fwd8_as<decltype(fast_tag)::value>(ga8, up8, h8);
        const uint4 ph = Vec8<IT>::pack(h8);
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4v, ph),
                                    reinterpret_cast<u32x4v*>(hb + oh[h] + kxb));
        uint4 pl = ph;  // what the products read
        if constexpr (DROP) {  // the dropout kernels' test and value on the stored h
          float hv[8], v[8];
          Vec8<IT>::unpack(ph, hv);
          const uint32_t base = (uint32_t)((uint64_t)rowc[h] * (uint64_t)K) + (uint32_t)kx;
          uint32_t b = 0;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const bool keep =
                ql_philox::keep_word(ql_philox::philox_word0(base + e, dr.seed), dr.thr);
            v[e] = keep ? hv[e] * dr.scale : 0.0f;
            b |= (uint32_t)keep << e;
          }
          pl = Vec8<IT>::pack(v);
          dr.bits[ql_philox::keep_byte(rowc[h], kx, dr.gs)] = (uint8_t)b;
        }
        *reinterpret_cast<uint4*>(lb + lds_w + 8 * h * kSwLdsRow) = pl;
      }
    };
    if (__builtin_expect(fast, 1)) rows(std::true_type{});
    else rows(std::false_type{});
    __syncthreads();
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        const uint4 f = *reinterpret_cast<const uint4*>(lb + lds_r + 16 * rg * kSwLdsRow +
                                                        64 * (2 * wave + gi));
        if (k0 + 32 * (2 * wave + gi) < ke) acc[rg][gi] = mfma<IT>(yv[gi], f, acc[rg][gi]);
      }
    }
    buf ^= 1;
  }
  // sum over the waves in wave order through LDS; wave rg < RG finishes row group rg
  __syncthreads();
  f32x4_t* red = reinterpret_cast<f32x4_t*>(lds);
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) red[(rg * 4 + wave) * 64 + lane] = acc[rg][0] + acc[rg][1];
  __syncthreads();
  const int cc = 4 * (lane >> 4);
  if (wave < RG) {
    const int64_t row = m0 + 16 * wave + (lane & 15);
    if (row < M) {
      f32x4_t sum = red[(wave * 4) * 64 + lane];
#pragma unroll
      for (int w = 1; w < 4; ++w) sum += red[(wave * 4 + w) * 64 + lane];
      if constexpr (PARTIAL) {
        *reinterpret_cast<float4*>(ws + ((int64_t)blockIdx.y * M + row) * kRank + cc) =
            make_float4(sum[0], sum[1], sum[2], sum[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint16_t v = Elem<IT>::from_f32(alpha * sum[e]);
          out[row * ldo + cc + e] = v;
          if (out_t) out_t[(int64_t)(cc + e) * ldt + row] = v;
        }
      }
    }
  }
  if constexpr (!PARTIAL) {
    const int64_t row = m0 + 16 * (3 - wave) + (lane & 15);  // waves 2, 3: the zero columns
    if (wave >= 4 - RG && row < M)
      for (int zc = kRank + cc; zc < out_cols; zc += 16)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (zc + e < out_cols) out[row * ldo + zc + e] = Elem<IT>::from_f32(0.f);
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

// Store 4 consecutive values (n, c .. c+3) of out [N, nc] (or of its transpose [nc, N]).
QL_DEV void store_wgrad4(float* __restrict__ out, bool out_t, int64_t N, int nc, int64_t n,
                         int64_t c, float4 v) {
  if (out_t) {
    out[(c + 0) * N + n] = v.x;
    out[(c + 1) * N + n] = v.y;
    out[(c + 2) * N + n] = v.z;
    out[(c + 3) * N + n] = v.w;
  } else {
    *reinterpret_cast<float4*>(out + n * nc + c) = v;
  }
}

// The lora_A gradients of adapters whose inputs are their own dropout masks of one shared Q
// (dA_g^T = du_g^T xd_g with xd_g = keep_g * (Q * scale rounded to Q's type)): the kernel
// reads Q once and each adapter's keep bits (8 x 8 blocks, ql_philox.h: one 8-byte word per
// lane's 8 x 8 block of Q), scales the block as the dropout kernels do, and zeroes the dropped
// rows of each transposed fragment before the adapter's products. The sums are those of
// lora_wgrad over the stored xd_g, in the same order.
typedef short s16x2_t __attribute__((ext_vector_type(2)));

// Q's 8 x 8 block times the dropout scale, rounded to the input type (the dropped input's value
// for a kept element).
template <int IT> QL_DEV void scale_block(uint4 (&q)[8], float scale) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float v[8];
    Vec8<IT>::unpack(q[i], v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = v[j] * scale;
    q[i] = Vec8<IT>::pack(v);
  }
}

// The keep bytes of a block's rows (w: row i in byte i) spread for transposed fragments: word p
// holds row 2p's byte in its low half and row 2p + 1's in its high half.
QL_DEV void spread_rows(const uint2& w, uint32_t (&sp)[4]) {
  sp[0] = __builtin_amdgcn_perm(w.x, w.x, 0x0C010C00u);
  sp[1] = __builtin_amdgcn_perm(w.x, w.x, 0x0C030C02u);
  sp[2] = __builtin_amdgcn_perm(w.y, w.y, 0x0C010C00u);
  sp[3] = __builtin_amdgcn_perm(w.y, w.y, 0x0C030C02u);
}

// Fragment T (column T of the block, rows 2p and 2p + 1 in word p) with the dropped rows zeroed:
// bit T of each half moves to the half's sign bit and an arithmetic shift makes it 0 or 0xFFFF.
template <int T> QL_DEV uint4 mask_column(const uint4& f, const uint32_t (&sp)[4]) {
  uint32_t m[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    s16x2_t v = __builtin_bit_cast(s16x2_t, sp[p]);
    v = (v << (short)(15 - T)) >> (short)15;
    m[p] = __builtin_bit_cast(uint32_t, v);
  }
  return make_uint4(f.x & m[0], f.y & m[1], f.z & m[2], f.w & m[3]);
}

// MFMAs of one 8 x 8 block (transposed fragments qt) with each adapter's P fragment, the
// adapter's keep word applied when MASKED.
template <int IT, int G, bool MASKED>
QL_DEV void wgrad_block(f32x4_t (&acc)[G][8], const uint4 (&qt)[8], const uint4 (&pf)[G],
                        const uint2 (&kw)[G]) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if constexpr (MASKED) {
      uint32_t sp[4];
      spread_rows(kw[g], sp);
      acc[g][0] = mfma<IT>(pf[g], mask_column<0>(qt[0], sp), acc[g][0]);
      acc[g][1] = mfma<IT>(pf[g], mask_column<1>(qt[1], sp), acc[g][1]);
      acc[g][2] = mfma<IT>(pf[g], mask_column<2>(qt[2], sp), acc[g][2]);
      acc[g][3] = mfma<IT>(pf[g], mask_column<3>(qt[3], sp), acc[g][3]);
      acc[g][4] = mfma<IT>(pf[g], mask_column<4>(qt[4], sp), acc[g][4]);
      acc[g][5] = mfma<IT>(pf[g], mask_column<5>(qt[5], sp), acc[g][5]);
      acc[g][6] = mfma<IT>(pf[g], mask_column<6>(qt[6], sp), acc[g][6]);
      acc[g][7] = mfma<IT>(pf[g], mask_column<7>(qt[7], sp), acc[g][7]);
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[g][t] = mfma<IT>(pf[g], qt[t], acc[g][t]);
    }
  }
}

// PARTIAL: each split writes its fp32 [N, NC] partial to ws[split]; lora_wgrad_reduce sums
// them in split order. (Summing inside this launch by the last workgroup of each column block
// needs device-scope release/acquire fences per workgroup, whose L2 write-back and invalidate
// cost more than the separate reduce launch.)
// U: 32-row chunks per wave per step of the main loop (the host picks one that divides the
// chunks of a split, so only a ragged last split reaches the single-chunk loops after it).
template <int IT, bool PARTIAL, int G, int U, bool MASKED>
__global__ __launch_bounds__(kThreads) void lora_wgrad_kernel(
    const uint16_t* __restrict__ PT, int64_t ldpt, const uint16_t* __restrict__ Q, int64_t ldq,
    int64_t M, int64_t N, int64_t m_per_split, float* __restrict__ ws, float* __restrict__ out,
    float alpha, bool out_t, WgradMask mk) {
  constexpr int NC = kRank * G;
  __shared__ f32x4_t red[4 * 8 * 64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cg = lane & 15;                 // column group: columns n0 + 8 cg .. +7
  const int mq = lane >> 4;                 // rows 8 mq .. 8 mq + 7 of a 32-row chunk
  const int64_t n0 = (int64_t)blockIdx.x * 128;
  const int64_t ncol = n0 + 8 * cg;
  const bool col_ok = ncol < N;             // N % 8 == 0: a group is all in or all out
  // Lanes past N read columns 0 .. 7 instead: output column j of an MFMA depends only on the
  // lanes that supply column j, and those sums are never stored.
  const int64_t ncolc = col_ok ? ncol : 0;
  const int64_t mb = (int64_t)blockIdx.y * m_per_split;
  const int64_t me = mb + m_per_split < M ? mb + m_per_split : M;
  const uint32_t qo = (uint32_t)(((int64_t)8 * mq * ldq + ncolc) * 2);
  const uint32_t ldq2 = (uint32_t)(ldq * 2);
  uint32_t po[G];  // row 16 g + cg of P^T (P[:, 16 g + cg], m-contiguous), rows 8 mq .. +7
#pragma unroll
  for (int g = 0; g < G; ++g) po[g] = (uint32_t)(((int64_t)(16 * g + cg) * ldpt + 8 * mq) * 2);
  f32x4_t acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[g][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Wave w takes the 32-row chunks mb + 32 w + 128 i; lane l loads rows 8 (l / 16) .. +7 of a
  // chunk at columns 8 (l % 16) .. +7 as eight 16-B row pieces (lanes 0-15 of a row read 256
  // contiguous bytes) and the matching 8 rows of P, transposes the block in registers into
  // eight fragments that each hold 8 consecutive rows of one column, and multiplies them by
  // P's fragment: MFMA t accumulates column n0 + 8 (l % 16) + t.
  // keep words: the 8-byte word of block (rows r .. r + 7, columns ncolc .. +7), r a multiple
  // of 8, is at r / 8 * gs + ncolc
  auto keep_words = [&](int64_t r, uint2 (&kw)[G]) {
#pragma unroll
    for (int g = 0; g < G; ++g)
      kw[g] = *reinterpret_cast<const uint2*>(mk.p[g] + (r >> 3) * mk.gs + ncolc);
  };
  int64_t m = mb + 32 * wave;
  for (; m + 128 * (U - 1) + 32 <= me; m += 128 * U) {  // U whole chunks: loads only
    uint4 q[U][8], pf[U][G];
    uint2 kw[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const char* qb = reinterpret_cast<const char*>(Q + (m + 128 * u) * ldq);
      const char* pb = reinterpret_cast<const char*>(PT + m + 128 * u);
#pragma unroll
      for (int g = 0; g < G; ++g) pf[u][g] = ld16(pb, po[g]);
#pragma unroll
      for (int i = 0; i < 8; ++i) q[u][i] = ld16(qb, qo + i * ldq2);
      if constexpr (MASKED) keep_words(m + 128 * u + 8 * mq, kw[u]);
    }
    __builtin_amdgcn_sched_barrier(0);  // the step's loads all go out before the first wait
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (MASKED) scale_block<IT>(q[u], mk.scale);
      uint4 qt[8];
      transpose8x8(q[u], qt);
      wgrad_block<IT, G, MASKED>(acc, qt, pf[u], kw[u]);
    }
  }
  for (; m + 32 <= me; m += 128) {  // whole chunks left (fewer than U), one at a time
    uint4 q[8], pf[G];
    uint2 kw[G];
    const char* qb = reinterpret_cast<const char*>(Q + m * ldq);
    const char* pb = reinterpret_cast<const char*>(PT + m);
#pragma unroll
    for (int g = 0; g < G; ++g) pf[g] = ld16(pb, po[g]);
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = ld16(qb, qo + i * ldq2);
    if constexpr (MASKED) {
      keep_words(m + 8 * mq, kw);
      scale_block<IT>(q, mk.scale);
    }
    uint4 qt[8];
    transpose8x8(q, qt);
    wgrad_block<IT, G, MASKED>(acc, qt, pf, kw);
  }
  if (m < me) {  // a partial chunk: rows past me contribute zeros
    const int64_t r0 = m + 8 * mq;
    uint4 q[8], pf[G];
    if (r0 + 8 <= me) {
#pragma unroll
      for (int g = 0; g < G; ++g)
        pf[g] = *reinterpret_cast<const uint4*>(PT + (int64_t)(16 * g + cg) * ldpt + r0);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        q[i] = *reinterpret_cast<const uint4*>(Q + (r0 + i) * ldq + ncolc);
    } else {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint16_t* pr = PT + (int64_t)(16 * g + cg) * ldpt;
        uint16_t pv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) pv[i] = r0 + i < me ? pr[r0 + i] : (uint16_t)0;
        pf[g] = make_uint4((uint32_t)pv[0] | ((uint32_t)pv[1] << 16),
                           (uint32_t)pv[2] | ((uint32_t)pv[3] << 16),
                           (uint32_t)pv[4] | ((uint32_t)pv[5] << 16),
                           (uint32_t)pv[6] | ((uint32_t)pv[7] << 16));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        q[i] = r0 + i < me ? *reinterpret_cast<const uint4*>(Q + (r0 + i) * ldq + ncolc)
                           : make_uint4(0, 0, 0, 0);
    }
    uint2 kw[G];
    if constexpr (MASKED) {
      // rows past me hold zeros; a block that starts past M has no keep word (nor anything to
      // mask)
      if (r0 < M) {
        keep_words(r0, kw);
      } else {
#pragma unroll
        for (int g = 0; g < G; ++g) kw[g] = make_uint2(0, 0);
      }
      scale_block<IT>(q, mk.scale);
    }
    uint4 qt[8];
    transpose8x8(q, qt);
    wgrad_block<IT, G, MASKED>(acc, qt, pf, kw);
  }
  // acc[g][t]: lane holds out[n = ncol + t][16 g + 4 (lane / 16) .. +3]. Per slot: every wave
  // writes its 8 accumulators, then wave w sums t = 2w, 2w + 1 over the waves in wave order.
  const int c = 4 * mq;
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int t = 0; t < 8; ++t) red[(wave * 8 + t) * 64 + lane] = acc[g][t];
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int t = 2 * wave + h;
      f32x4_t s = red[t * 64 + lane];
#pragma unroll
      for (int w = 1; w < 4; ++w) s += red[(w * 8 + t) * 64 + lane];
      if (col_ok) {
        const int64_t n = ncol + t;
        if constexpr (PARTIAL) {
          *reinterpret_cast<float4*>(ws + ((int64_t)blockIdx.y * N + n) * NC + kRank * g + c) =
              make_float4(s[0], s[1], s[2], s[3]);
        } else {
          store_wgrad4(out, out_t, N, NC, n, kRank * g + c,
                       make_float4(alpha * s[0], alpha * s[1], alpha * s[2], alpha * s[3]));
        }
      }
    }
    __syncthreads();
  }
}

// out = alpha * sum over splits of ws[split] ([N, nc] fp32 each); splits = 0 writes zeros.
// 64 float4 outputs per workgroup: wave w sums splits [w S / 4, (w + 1) S / 4) in split order
// (all of its loads for an output in flight together, 4 at a time), and wave 0 adds the other
// waves' sums in wave order, so the result does not depend on the launch shape.
QL_DEV void wgrad_reduce_body(const float* __restrict__ ws, int splits, int64_t N, int nc,
                              float* __restrict__ out, float alpha, bool out_t,
                              float4 (*__restrict__ part)[64]) {
  const int64_t total4 = N * nc / 4;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int z0 = splits * w / 4, z1 = splits * (w + 1) / 4;
  for (int64_t base = (int64_t)blockIdx.x * 64; base < total4; base += (int64_t)gridDim.x * 64) {
    const int64_t i = base + lane;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < total4) {
      const float4* w4 = reinterpret_cast<const float4*>(ws) + i;
      int z = z0;
      for (; z + 4 <= z1; z += 4) {
        float4 t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = w4[(int64_t)(z + j) * total4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v.x += t[j].x; v.y += t[j].y; v.z += t[j].z; v.w += t[j].w;
        }
      }
      for (; z < z1; ++z) {
        const float4 t = w4[(int64_t)z * total4];
        v.x += t.x; v.y += t.y; v.z += t.z; v.w += t.w;
      }
    }
    if (w > 0) part[w - 1][lane] = v;
    __syncthreads();
    if (w == 0 && i < total4) {
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const float4 t = part[q][lane];
        v.x += t.x; v.y += t.y; v.z += t.z; v.w += t.w;
      }
      const int64_t n = (4 * i) / nc, c = 4 * i - n * nc;
      store_wgrad4(out, out_t, N, nc, n, c, make_float4(alpha * v.x, alpha * v.y, alpha * v.z,
                                                        alpha * v.w));
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void lora_wgrad_reduce(const float* __restrict__ ws, int splits,
                                                         int64_t N, int nc,
                                                         float* __restrict__ out, float alpha,
                                                         bool out_t) {
  __shared__ float4 part[3][64];
  wgrad_reduce_body(ws, splits, N, nc, out, alpha, out_t, part);
}

// Up to three such reductions of one shape in one launch (blockIdx.y picks the product), each
// summed exactly as lora_wgrad_reduce sums it: the weight gradients one fused kernel leaves as
// partials (the SwiGLU backward's two lora_B and one lora_A), without a launch each.
struct WgradReduceSet {
  const float* ws[3];
  float* out[3];
  float alpha[3];
  bool out_t[3];
};

__global__ __launch_bounds__(256) void lora_wgrad_reduce_set(WgradReduceSet set, int splits,
                                                             int64_t N, int nc) {
  __shared__ float4 part[3][64];
  const int q = blockIdx.y;
  wgrad_reduce_body(set.ws[q], splits, N, nc, set.out[q], set.alpha[q], set.out_t[q], part);
}

// The diagonal blocks of a multi-slot weight gradient: out[n, c] = alpha_q * sum over splits
// (in split order) of ws[split][n][16 q + c], for the slot q whose columns [off_q, off_{q+1})
// hold n. With Q the concatenated output gradient of several adapters and P^T their stacked
// u^T, that is each adapter's lora_B gradient s_q g_q^T u_q, stacked as [N, 16].
struct WgradDiag {
  int64_t off[kMaxSlots + 1];
  float alpha[kMaxSlots];
  int slots;
};

__global__ __launch_bounds__(256) void lora_wgrad_reduce_diag(const float* __restrict__ ws,
                                                              int splits, int64_t N,
                                                              const WgradDiag d,
                                                              float* __restrict__ out) {
  const int nc = kRank * d.slots;
  const int64_t total4 = N * kRank / 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total4;
       i += (int64_t)gridDim.x * 256) {
    const int64_t n = (4 * i) / kRank, c = 4 * i - n * kRank;
    int q = 0;
    while (q + 1 < d.slots && n >= d.off[q + 1]) ++q;
    const float* src = ws + n * nc + kRank * q + c;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int z = 0; z < splits; ++z) {
      const float4 t = *reinterpret_cast<const float4*>(src + (int64_t)z * N * nc);
      v.x += t.x; v.y += t.y; v.z += t.z; v.w += t.w;
    }
    const float a = d.alpha[q];
    reinterpret_cast<float4*>(out)[i] = make_float4(a * v.x, a * v.y, a * v.z, a * v.w);
  }
}

// The compute-dtype forms of one adapter's fp32 factors A [16, K] and B [N, 16], in one pass:
//   a16 [16, K]  = A                    (the Y operand of u = x A^T)
//   at  [K, 64]  = A^T | 0              (the second K segment of the backward dX GEMM)
//   bs  [N, 64]  = s B | 0              (the second K segment of the forward GEMM)
//   bt  [16, N]  = B^T                  (the Y operand of du = s g B)
// Thread t of the flat range handles one row of at (t < K), then one row of bs and one
// column of bt (K <= t < K + N), then 8 elements of a16. qlora_lora_pack uses this form only
// for a pad that is not a multiple of 8 or rows that are not 16-B aligned; otherwise it runs
// the one-slot group packing, which writes whole 16-B chunks.
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
// outputs. The padded rows of at and bs are written one 16-B chunk per work item, so the 8
// consecutive lanes of one 128-B row (pad 64) write it whole and every item needs one round of
// loads; a thread per row walking its chunks (or storing 2 B per column) cost 6-8 us per launch
// at the 7B shapes, almost all of it store issue and serial load waits. Work items, in order:
//   [0, K ch)            chunk t % ch of row t / ch of at  (ch = pad / 8)
//   [.., + N ch)         the same for the rows of bs
//   [.., + N)            column n of bt (every slot's 16 rows)
//   then 8 elements of a16 per item.
constexpr int kMaxGroup = 4;
struct PackGroupArgs {
  const float* A[kMaxGroup];  // [16, K]
  const float* B[kMaxGroup];  // [n_g, 16]
  float scale[kMaxGroup];
  int64_t off[kMaxGroup + 1];  // prefix sums of n_g
  int G;
};

// The work items t0, t0 + stride, ... of one group's packing; `p` may live in the kernel
// arguments or in LDS (indexed by the item's slot either way).
template <int OT, typename Args>
QL_DEV void pack_group_items(const Args& p, int64_t K, typename Elem<OT>::T* __restrict__ a16,
                             typename Elem<OT>::T* __restrict__ at,
                             typename Elem<OT>::T* __restrict__ bs,
                             typename Elem<OT>::T* __restrict__ bt, int pad, int64_t t0,
                             int64_t stride) {
  const int64_t N = p.off[p.G];
  const int ch = pad / 8;
  const int64_t n_at = K * ch, n_bs = N * ch;
  const int64_t n_a16 = (int64_t)kRank * p.G * K / 8;
  const int64_t total = n_at + n_bs + N + n_a16;
  auto slot_of = [&](int64_t n) {
    int g = 0;
    while (g + 1 < p.G && n >= p.off[g + 1]) ++g;
    return g;
  };
  for (int64_t t = t0; t < total; t += stride) {
    if (t < n_at) {
      // at [K, pad]: column 16 g + r of row k holds A_g[r][k]
      const int64_t k = t / ch;
      const int c0 = 8 * (int)(t - k * ch);
      const int g = c0 / kRank;
      float v[8];
      if (g < p.G) {
        const float* a = p.A[g] + (int64_t)(c0 & (kRank - 1)) * K + k;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = a[(int64_t)e * K];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.f;
      }
      Vec8<OT>::store(at + k * pad + c0, v);
    } else if (t < n_at + n_bs) {
      // bs [N, pad]: row n of slot g holds scale_g B_g[n - off_g] in columns 16 g .. 16 g + 15
      const int64_t u = t - n_at;
      const int64_t n = u / ch;
      const int c0 = 8 * (int)(u - n * ch);
      const int g = slot_of(n);
      float v[8];
      if (c0 / kRank == g) {
        const float* b = p.B[g] + (n - p.off[g]) * kRank + (c0 & (kRank - 1));
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = p.scale[g] * b[e];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.f;
      }
      Vec8<OT>::store(bs + n * pad + c0, v);
    } else if (t < n_at + n_bs + N) {
      // bt [16 G, N] block-diagonal: column n holds B_g^T in rows 16 g .. 16 g + 15 and zeros
      // in the other slots' rows, so one multi-slot lora_down over all N columns gives every
      // adapter's du at once
      const int64_t n = t - n_at - n_bs;
      const int g = slot_of(n);
      float b[kRank];
#pragma unroll
      for (int r = 0; r < kRank; ++r) b[r] = p.B[g][(n - p.off[g]) * kRank + r];
      for (int q = 0; q < p.G; ++q)
#pragma unroll
        for (int r = 0; r < kRank; ++r)
          bt[(int64_t)(kRank * q + r) * N + n] = Elem<OT>::from_f32(q == g ? b[r] : 0.f);
    } else {
      const int64_t i = (t - n_at - n_bs - N) * 8;  // into a16 [16 G, K]
      const int64_t gr = i / K, col = i - gr * K;
      const int g = (int)(gr / kRank), r = (int)(gr - (int64_t)g * kRank);
#pragma unroll
      for (int e = 0; e < 8; ++e) a16[i + e] = Elem<OT>::from_f32(p.A[g][(int64_t)r * K + col + e]);
    }
  }
}

template <int OT>
__global__ __launch_bounds__(256) void lora_pack_group_kernel(PackGroupArgs p, int64_t K,
                                                              typename Elem<OT>::T* __restrict__ a16,
                                                              typename Elem<OT>::T* __restrict__ at,
                                                              typename Elem<OT>::T* __restrict__ bs,
                                                              typename Elem<OT>::T* __restrict__ bt,
                                                              int pad) {
  pack_group_items<OT>(p, K, a16, at, bs, bt, pad, (int64_t)blockIdx.x * 256 + threadIdx.x,
                       (int64_t)gridDim.x * 256);
}

static_assert(sizeof(ql_lora_pack_job) == 160, "ql_lora_pack_job layout");

// Many groups' packings in one launch: blockIdx.y selects the job (a descriptor in device
// memory, copied to LDS once per workgroup), blockIdx.x strides over its work items.
template <int OT>
__global__ __launch_bounds__(256) void lora_pack_jobs_kernel(const ql_lora_pack_job* __restrict__ jobs,
                                                             char* __restrict__ base, int pad) {
  using T = typename Elem<OT>::T;
  __shared__ PackGroupArgs p;
  __shared__ int64_t sK, so[4];
  if (threadIdx.x == 0) {
    const ql_lora_pack_job& j = jobs[blockIdx.y];
    p.G = j.count;
    p.off[0] = 0;
    for (int g = 0; g < kMaxGroup; ++g) {
      const bool in = g < j.count;
      p.A[g] = in ? j.A[g] : nullptr;
      p.B[g] = in ? j.B[g] : nullptr;
      p.scale[g] = in ? j.scaling[g] : 0.f;
      p.off[g + 1] = p.off[g] + (in ? j.n[g] : 0);
    }
    sK = j.K;
    so[0] = j.a16;
    so[1] = j.at_pad;
    so[2] = j.bs_pad;
    so[3] = j.bt;
  }
  __syncthreads();
  pack_group_items<OT>(p, sK, reinterpret_cast<T*>(base + so[0]), reinterpret_cast<T*>(base + so[1]),
                       reinterpret_cast<T*>(base + so[2]), reinterpret_cast<T*>(base + so[3]), pad,
                       (int64_t)blockIdx.x * 256 + threadIdx.x, (int64_t)gridDim.x * 256);
}

// ---------------------------------------------------------------------------------------
// LoRA dropout fused with the adapters' down-projections (the forward with p > 0) for the
// G <= 4 adapters of a group that read one input, each with its own mask and seed:
//   xd_g = x * keep_g * scale (rounded to the input type)   stored when asked for (XD)
//   keep_g                                                   stored as bits (8 x 8 blocks):
//                                                            the backward's dx and lora_A
//                                                            gradient passes read them with x
//   u[m, 16 g + c] = sum_k xd_g[m, k] A[16 g + c, k]
// in one pass over x. keep_g is the Philox test of ql_philox.h at flat index m * K + k with
// seed_g, computed as the dropout kernels compute it, so xd_g and bits_g equal theirs bit for
// bit. A workgroup of 8 waves takes 16 rows and a range of 64-k chunks (blockIdx.y: the K
// split); wave w walks chunks w, w + 8, ... of the range. Lane l
// holds row l % 16 and k = 64 j + 32 h + 8 (l / 16) .. +7 (h = 0, 1), the v_mfma_f32_16x16x32
// operand layout, so the dropped values reach the matrix cores from the registers that formed
// them; each adapter's A fragment for the same k comes from L2. The waves' sums are added
// through LDS in wave order, the splits' by lora_down_reduce in split order (deterministic).
// Like the dropout kernels, the kernel is bound by the Philox rounds' integer multiplies; the
// products and the stores ride along. The K split is there for occupancy: the rounds of one
// element are a dependent chain, and a workgroup per 16 rows alone leaves two waves a SIMD.
constexpr int kDdWaves = 8;

// 16 B of lane src_byte / 4's fragment h0 or h1 (hi), moved with one ds_bpermute per dword
// and fragment.
QL_DEV uint4 from_fragments(const uint4& h0, const uint4& h1, int src_byte, bool hi) {
  const uint4 a = to_mfma_layout(h0, src_byte);
  const uint4 b = to_mfma_layout(h1, src_byte);
  return hi ? b : a;
}

struct DropDownSlots {
  uint64_t seed[kMaxSlots];
  uint16_t* xd[kMaxSlots];  // [M, >= K] with one row stride for all slots
  uint8_t* bits[kMaxSlots]; // 8 x 8 blocks (ql_philox.h), one group stride for all slots
};

template <int DT, int G, bool PARTIAL, bool XD>
__global__ __launch_bounds__(64 * kDdWaves) void dropout_down_kernel(
    const uint16_t* __restrict__ X, int64_t ldx, const uint16_t* __restrict__ A, int64_t lda,
    int64_t M, int64_t K, int64_t chunks_per_split, DropDownSlots sl, int64_t xd_rs,
    int64_t bits_gs, uint32_t thr, float scale, float* __restrict__ ws,
    uint16_t* __restrict__ out, int64_t ldo, int out_cols, uint16_t* __restrict__ out_t,
    int64_t ldt) {
  __shared__ f32x4_t red[G * kDdWaves * 64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int64_t row = (int64_t)blockIdx.x * 16 + r;
  const bool live = row < M;
  // Lanes of rows past M redo row M - 1 (its x, its counters, its stores of the same values),
  // so the loop's stores need no branch: a branch around them makes the wait-count pass assume
  // the path without stores and wait for every store before the next chunk's loads.
  const int64_t srow = live ? row : M - 1;
  const uint16_t* xr = X + srow * ldx + 8 * q;
  const uint16_t* ar = A + (int64_t)r * lda + 8 * q;
  // store layout (see the stores below): lane l writes row 8 t + l / 8 of the block, taken from
  // the fragment lane of that row and k group (l % 8) & 3, fragment h = (l % 8) / 4
  int perm_src[2];
  int64_t srow_t[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    perm_src[t] = 4 * (8 * t + (lane >> 3) + 16 * (lane & 3));  // ds_bpermute byte address
    const int64_t tr = (int64_t)blockIdx.x * 16 + 8 * t + (lane >> 3);
    srow_t[t] = tr < M ? tr : M - 1;  // the source lane redid row M - 1 for rows past M
  }
  const bool perm_hi = (lane >> 2) & 1;
  // the reference's offsets are int32 (row * K + k): the counter is their low 32 bits
  const uint32_t flat_row = (uint32_t)((uint64_t)srow * (uint64_t)K) + 8u * (uint32_t)q;
  f32x4_t acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int64_t jb = (int64_t)blockIdx.y * chunks_per_split;
  const int64_t je = jb + chunks_per_split < K / 64 ? jb + chunks_per_split : K / 64;
  // One chunk of loads in flight ahead of the arithmetic: the next chunk's x and A fragments
  // are issued before this chunk's stores, so waiting for them never waits for the stores
  // (vmcnt counts loads and stores in issue order). The last chunk reloads itself.
  uint4 xv[2], av[G][2];
  auto load_chunk = [&](int64_t j, uint4 (&xo)[2], uint4 (&ao)[G][2]) {
    const int64_t c0 = 64 * j;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      xo[h] = *reinterpret_cast<const uint4*>(xr + c0 + 32 * h);
#pragma unroll
      for (int g = 0; g < G; ++g)
        ao[g][h] = *reinterpret_cast<const uint4*>(ar + (int64_t)16 * g * lda + c0 + 32 * h);
    }
  };
  const int64_t j0 = jb + wave;
  if (j0 < je) load_chunk(j0, xv, av);
  for (int64_t j = j0; j < je; j += kDdWaves) {
    uint4 xn[2], an[G][2];
    load_chunk(j + kDdWaves < je ? j + kDdWaves : j, xn, an);
    // keep the next chunk's loads ahead of this chunk's stores (the scheduler would sink them
    // past the arithmetic, after the stores, and the next wait would then cover the stores)
    __builtin_amdgcn_sched_barrier(0);
    const int64_t c0 = 64 * j;
    float xf[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h) Vec8<DT>::unpack(xv[h], xf[h]);
    const int64_t c = c0 + 8 * (lane & 7);
#pragma unroll
    for (int g = 0; g < G; ++g) {  // one adapter at a time: its mask, product and stores
      uint4 dv[2];
      uint32_t bw[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t base = flat_row + (uint32_t)(c0 + 32 * h);
        float v[8];
        uint32_t b = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const bool keep = ql_philox::keep_word(ql_philox::philox_word0(base + e, sl.seed[g]), thr);
          v[e] = keep ? xf[h][e] * scale : 0.0f;
          b |= (uint32_t)keep << e;
        }
        dv[h] = Vec8<DT>::pack(v);
        bw[h] = b;
      }
      acc[g] = mfma<DT>(av[g][0], dv[0], acc[g]);
      acc[g] = mfma<DT>(av[g][1], dv[1], acc[g]);
      // Stores: lane permutes turn the two fragments (16 rows x 32 k each) into two
      // row-major 8 x 64 tiles, lane l holding row 8 t + l / 8, k = c0 + 8 (l % 8) .. +7, so
      // each store instruction writes 8 whole 128-B row pieces instead of 16 half lines.
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        uint4 o{};
        if constexpr (XD) o = from_fragments(dv[0], dv[1], perm_src[t], perm_hi);
        const uint32_t b0 = (uint32_t)__builtin_amdgcn_ds_bpermute(perm_src[t], (int)bw[0]);
        const uint32_t b1 = (uint32_t)__builtin_amdgcn_ds_bpermute(perm_src[t], (int)bw[1]);
        if constexpr (XD) *reinterpret_cast<uint4*>(sl.xd[g] + srow_t[t] * xd_rs + c) = o;
        // 8 x 8 block layout: the 64 lanes' bytes are 64 contiguous bytes
        sl.bits[g][ql_philox::keep_byte(srow_t[t], c, bits_gs)] = (uint8_t)(perm_hi ? b1 : b0);
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      xv[h] = xn[h];
#pragma unroll
      for (int g = 0; g < G; ++g) av[g][h] = an[g][h];
    }
  }
  // acc[g]: lane l holds u[row m0 + l % 16][16 g + 4 (l / 16) .. +3] of this wave's chunks
#pragma unroll
  for (int g = 0; g < G; ++g) red[(g * kDdWaves + wave) * 64 + lane] = acc[g];
  __syncthreads();
  if (!live) return;
  const int c = 4 * q;
  using T = typename Elem<DT>::T;
  if (wave < G) {  // wave g finishes slot g
    const int g = wave;
    f32x4_t s = red[g * kDdWaves * 64 + lane];
#pragma unroll
    for (int w = 1; w < kDdWaves; ++w) s += red[(g * kDdWaves + w) * 64 + lane];
    const int col = kRank * g + c;
    if constexpr (PARTIAL) {  // this split's sums, added in split order by lora_down_reduce
      *reinterpret_cast<float4*>(ws + ((int64_t)blockIdx.y * M + row) * (kRank * G) + col) =
          make_float4(s[0], s[1], s[2], s[3]);
      return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) out[row * ldo + col + e] = Elem<DT>::from_f32(s[e]);
    if (out_t) {
#pragma unroll
      for (int e = 0; e < 4; ++e) out_t[(int64_t)(col + e) * ldt + row] = Elem<DT>::from_f32(s[e]);
    }
  } else if (!PARTIAL && wave == kDdWaves - 1) {  // the zero columns 16 G .. out_cols - 1
    for (int zc = kRank * G + c; zc < out_cols; zc += 16)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (zc + e < out_cols) out[row * ldo + zc + e] = (T)0;
  }
}

unsigned grid1d(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 4096) g = 4096;
  return (unsigned)(g > 0 ? g : 1);
}
// lora_wgrad_reduce: 64 outputs per workgroup
unsigned grid64(int64_t n) {
  int64_t g = (n + 63) / 64;
  if (g > 4096) g = 4096;
  return (unsigned)(g > 0 ? g : 1);
}

}  // namespace

// ---- host side -------------------------------------------------------------------------

// 16-row groups per workgroup: 4 for a long single-adapter reduction (each fragment of Y then
// serves four of X; the K split below restores the workgroup count), else 1.
static int lora_down_rows(int64_t M, int64_t K, int slots) {
  return (slots == 1 && K >= 8192 && M >= 1024) ? 4 : 1;
}

// Split K only while there are fewer than 256 row blocks (one workgroup per CU is enough to
// stream X at full bandwidth with a few 128-k chunks in flight per wave), keeping at least
// two chunks per wave in each split.
int ql_lora_down_splits(int64_t M, int64_t K, int slots) {
  const int64_t rows = 16 * lora_down_rows(M, K, slots);
  const int64_t blocks = (M + rows - 1) / rows;
  int s = 1;
  while (blocks * s < 256 && K / (128 * kDownWaves * 2 * s) >= 1 && s < 64) s *= 2;
  return s;
}

int64_t ql_lora_down_workspace_floats(int64_t M, int64_t K, int slots) {
  const int s = ql_lora_down_splits(M, K, slots);
  return s > 1 ? (int64_t)s * M * kRank * slots : 0;
}

int ql_lora_down(int in_dtype, int out_dtype, const void* X, int64_t ldx, const void* Y,
                 int64_t ldy, int64_t M, int64_t K, int slots, void* out, int64_t ldo,
                 int out_cols, float alpha, void* out_t, int64_t ldt, float* ws,
                 int64_t ws_floats, hipStream_t s) {
  if (slots < 1 || slots > kMaxSlots) return QL_EINVAL;
  const int nc = kRank * slots;
  if (M <= 0 || K <= 0 || K % 32 || out_cols < nc || ldo < out_cols) return QL_EINVAL;
  if (out_t && ldt < M) return QL_EINVAL;
  if (ldx % 8 || ldy % 8 || !ql_aligned(X, 16) || !ql_aligned(Y, 16)) return QL_EALIGN;
  // per-lane byte offsets within a workgroup's 16 * rows rows of X and within Y are 32-bit
  const int rows = lora_down_rows(M, K, slots);
  if (ldx < K || ldy < K || 32 * rows * ldx >= (int64_t(1) << 31) ||
      2 * nc * ldy >= (int64_t(1) << 31))
    return QL_EINVAL;
  if (in_dtype != QL_BF16 && in_dtype != QL_F16) return QL_EDTYPE;
  if (out_dtype != QL_BF16 && out_dtype != QL_F16 && out_dtype != QL_F32) return QL_EDTYPE;
  int splits = ql_lora_down_splits(M, K, slots);
  if (ws_floats < (int64_t)splits * M * nc || !ws) splits = 1;
  // per-split K range: a multiple of 128 k per wave
  constexpr int64_t kq = 128 * kDownWaves;
  int64_t kps = ((K + splits - 1) / splits + kq - 1) / kq * kq;
  splits = (int)((K + kps - 1) / kps);
  const dim3 grid((unsigned)((M + 16 * rows - 1) / (16 * rows)), (unsigned)splits);
#define QL_DOWN_GR(IT, OT, G, R)                                                              \
  do {                                                                                        \
    using T = typename Elem<OT>::T;                                                           \
    if (splits == 1) {                                                                        \
      hipLaunchKernelGGL((lora_down_kernel<IT, OT, false, G, R>), grid, dim3(64 * kDownWaves), \
                         0, s, (const uint16_t*)X, ldx, (const uint16_t*)Y, ldy, M, K, kps,   \
                         (float*)nullptr, (T*)out, ldo, out_cols, alpha, (uint16_t*)out_t,    \
                         ldt);                                                                \
    } else {                                                                                  \
      hipLaunchKernelGGL((lora_down_kernel<IT, OT, true, G, R>), grid, dim3(64 * kDownWaves),  \
                         0, s, (const uint16_t*)X, ldx, (const uint16_t*)Y, ldy, M, K, kps,   \
                         ws, (T*)out, ldo, out_cols, alpha, (uint16_t*)out_t, ldt);           \
      hipLaunchKernelGGL((lora_down_reduce<IT, OT>), dim3(grid1d(M * out_cols)), dim3(256),   \
                         0, s, ws, splits, M, nc, (T*)out, ldo, out_cols, alpha, alpha,       \
                         (uint16_t*)out_t, ldt);                                              \
    }                                                                                         \
  } while (0)
#define QL_DOWN(IT, OT)                                   \
  do {                                                    \
    switch (slots) {                                      \
      case 1:                                             \
        if (rows == 4) QL_DOWN_GR(IT, OT, 1, 4);          \
        else QL_DOWN_GR(IT, OT, 1, 1);                    \
        break;                                            \
      case 2: QL_DOWN_GR(IT, OT, 2, 1); break;            \
      case 3: QL_DOWN_GR(IT, OT, 3, 1); break;            \
      default: QL_DOWN_GR(IT, OT, 4, 1); break;           \
    }                                                     \
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
#undef QL_DOWN_GR
  return ql_launch_status();
}

// Split the token range until there are at least 256 workgroups, keeping at least one whole
// 32-row chunk per wave in each split; while splits keep 2048 or more rows, go on to 512 (two
// workgroups per CU: with one, nothing overlaps a wave's wait for its step's loads; the
// 4096 x 18944 reduction went from 39 to 35 us with cold inputs).
int ql_lora_wgrad_splits(int64_t M, int64_t N, int slots) {
  (void)slots;
  const int64_t blocks = (N + 127) / 128;
  int s = 1;
  while ((blocks * s < 256 || (blocks * s < 512 && M / s >= 2048)) && M >= 128 * 2 * s &&
         s < 64)
    s *= 2;
  return s;
}

int64_t ql_lora_wgrad_workspace_floats(int64_t M, int64_t N, int slots) {
  const int s = ql_lora_wgrad_splits(M, N, slots);
  return s > 1 ? (int64_t)s * N * kRank * slots : 0;
}

int ql_lora_wgrad(int in_dtype, const void* PT, int64_t ldpt, const void* Q, int64_t ldq,
                  int64_t M, int64_t N, int slots, float* out, int out_t, float alpha, float* ws,
                  int64_t ws_floats, hipStream_t s, const WgradMask* mask) {
  if (slots < 1 || slots > kMaxSlots) return QL_EINVAL;
  const int nc = kRank * slots;
  if (M <= 0 || N <= 0 || N % 8 || ldpt < M || ldq < N) return QL_EINVAL;
  // per-lane byte offsets within 32 rows of Q and within P^T are 32-bit
  if (64 * ldq >= (int64_t(1) << 31) || 2 * nc * ldpt >= (int64_t(1) << 31)) return QL_EINVAL;
  if (ldq % 8 || ldpt % 8 || !ql_aligned(Q, 16) || !ql_aligned(PT, 16) || !ql_aligned(out, 16))
    return QL_EALIGN;
  if (out_t != 0 && out_t != 1) return QL_EINVAL;
  if (in_dtype != QL_BF16 && in_dtype != QL_F16) return QL_EDTYPE;
  int splits = ql_lora_wgrad_splits(M, N, slots);
  if (ws_floats < (int64_t)splits * N * nc || !ws) splits = 1;
  int64_t mps = ((M + splits - 1) / splits + 127) / 128 * 128;
  splits = (int)((M + mps - 1) / mps);
  const dim3 grid((unsigned)((N + 127) / 128), (unsigned)splits);
  // chunks per wave per step: the largest of 4 (one slot) or 2 (several; their accumulators
  // take the registers) that divides a split's mps / 128 chunks per wave. With a mask, 2 for
  // one slot too: the scaling and masking between the loads and the products want the
  // registers (4096 x 18944: 36.8 us against 45.1 at 4).
  const int64_t per_wave = mps / 128;
  const int unroll =
      (!mask && slots == 1 && per_wave % 4 == 0) ? 4 : (per_wave % 2 == 0 ? 2 : 1);
  const WgradMask mk = mask ? *mask : WgradMask{};
#define QL_WGRAD_GUM(IT, G, U, MK)                                                            \
  do {                                                                                        \
    if (splits == 1) {                                                                        \
      hipLaunchKernelGGL((lora_wgrad_kernel<IT, false, G, U, MK>), grid, dim3(kThreads), 0, s, \
                         (const uint16_t*)PT, ldpt, (const uint16_t*)Q, ldq, M, N, mps,       \
                         (float*)nullptr, out, alpha, out_t, mk);                             \
    } else {                                                                                  \
      hipLaunchKernelGGL((lora_wgrad_kernel<IT, true, G, U, MK>), grid, dim3(kThreads), 0, s,  \
                         (const uint16_t*)PT, ldpt, (const uint16_t*)Q, ldq, M, N, mps, ws,   \
                         out, alpha, out_t, mk);                                              \
      hipLaunchKernelGGL(lora_wgrad_reduce, dim3(grid64(N * nc / 4)), dim3(256), 0, s, ws,    \
                         splits, N, nc, out, alpha, out_t);                                   \
    }                                                                                         \
  } while (0)
#define QL_WGRAD_GU(IT, G, U)                          \
  do {                                                 \
    if (mask) QL_WGRAD_GUM(IT, G, U, true);            \
    else QL_WGRAD_GUM(IT, G, U, false);                \
  } while (0)
#define QL_WGRAD_G(IT, G)                                          \
  do {                                                             \
    if (unroll == 4) QL_WGRAD_GU(IT, G, (G == 1 ? 4 : 2));         \
    else if (unroll == 2) QL_WGRAD_GU(IT, G, 2);                   \
    else QL_WGRAD_GU(IT, G, 1);                                    \
  } while (0)
#define QL_WGRAD(IT)                         \
  do {                                       \
    switch (slots) {                         \
      case 1: QL_WGRAD_G(IT, 1); break;      \
      case 2: QL_WGRAD_G(IT, 2); break;      \
      case 3: QL_WGRAD_G(IT, 3); break;      \
      default: QL_WGRAD_G(IT, 4); break;     \
    }                                        \
  } while (0)
  if (in_dtype == QL_BF16) QL_WGRAD(QL_BF16);
  else QL_WGRAD(QL_F16);
#undef QL_WGRAD
#undef QL_WGRAD_G
#undef QL_WGRAD_GU
#undef QL_WGRAD_GUM
  return ql_launch_status();
}

// SwiGLU backward + the two down-projections: kSwRows rows per workgroup, K split until
// every CU has a workgroup (keeping at least two tiles per split).
int ql_swiglu_bwd_down_splits(int64_t M, int64_t K) {
  const int64_t blocks = (M + kSwRows - 1) / kSwRows;
  int s = 1;
  while (blocks * s < 256 && K / (kSwK * 2 * s) >= 1 && s < 64) s *= 2;
  return s;
}

// The forward with the down adapter's dropout draws one Philox word per element of h: its
// rounds are a dependent chain per element, so it wants more waves than the one a SIMD that
// 256 workgroups give. Split K until about four workgroups a CU (1024), keeping a tile per
// split.
int ql_swiglu_fwd_down_splits(int64_t M, int64_t K, bool drop) {
  if (!drop) return ql_swiglu_bwd_down_splits(M, K);
  const int64_t blocks = (M + kSwRows - 1) / kSwRows;
  int s = 1;
  while (blocks * s < 1024 && K / (kSwK * 2 * s) >= 1 && s < 64) s *= 2;
  return s;
}

static bool rows16_ok(const void* p, int64_t ld) { return ql_aligned(p, 16) && ld % 8 == 0; }

int ql_swiglu_bwd_down(int dtype, const void* GR, int64_t ldgr, const void* GA, int64_t ldga,
                       const void* UP, int64_t ldup, void* DG, int64_t lddg, void* DU,
                       int64_t lddu, int64_t M, int64_t K, const void* YG, const void* YU,
                       int64_t ldy, float alpha_g, float alpha_u, void* out, int64_t ldo,
                       int out_cols, void* out_t, int64_t ldt, float* ws, int64_t ws_floats,
                       hipStream_t s) {
  constexpr int NC = 2 * kRank;
  if (M <= 0 || K <= 0 || K % 32 || out_cols < NC || ldo < out_cols) return QL_EINVAL;
  if (out_t && ldt < M) return QL_EINVAL;
  if (ldgr < K || ldga < K || ldup < K || lddg < K || lddu < K || ldy < K) return QL_EINVAL;
  // per-lane byte offsets within a workgroup's rows are 32-bit
  const int64_t lim = int64_t(1) << 31;
  if (2 * kSwRows * (ldgr > ldga ? (ldgr > ldup ? ldgr : ldup) : (ldga > ldup ? ldga : ldup)) >= lim ||
      2 * kSwRows * (lddg > lddu ? lddg : lddu) >= lim || 32 * ldy >= lim)
    return QL_EINVAL;
  if (!rows16_ok(GR, ldgr) || !rows16_ok(GA, ldga) || !rows16_ok(UP, ldup) ||
      !rows16_ok(DG, lddg) || !rows16_ok(DU, lddu) || !rows16_ok(YG, ldy) || !rows16_ok(YU, ldy))
    return QL_EALIGN;
  if (dtype != QL_BF16 && dtype != QL_F16) return QL_EDTYPE;
  int splits = ql_swiglu_bwd_down_splits(M, K);
  if (ws_floats < (int64_t)splits * M * NC || !ws) splits = 1;
  int64_t kps = ((K + splits - 1) / splits + kSwK - 1) / kSwK * kSwK;
  splits = (int)((K + kps - 1) / kps);
  const dim3 grid((unsigned)((M + kSwRows - 1) / kSwRows), (unsigned)splits);
#define QL_SWD(IT)                                                                            \
  do {                                                                                        \
    if (splits == 1) {                                                                        \
      hipLaunchKernelGGL((swiglu_bwd_down_kernel<IT, false>), grid, dim3(256), 0,              \
                         s, (const uint16_t*)GR, ldgr, (const uint16_t*)GA, ldga,             \
                         (const uint16_t*)UP, ldup, (uint16_t*)DG, lddg, (uint16_t*)DU, lddu, \
                         (const uint16_t*)YG, (const uint16_t*)YU, ldy, M, K, kps,            \
                         (float*)nullptr, (uint16_t*)out, ldo, out_cols, alpha_g, alpha_u,    \
                         (uint16_t*)out_t, ldt);                                              \
    } else {                                                                                  \
      hipLaunchKernelGGL((swiglu_bwd_down_kernel<IT, true>), grid, dim3(256), 0,               \
                         s, (const uint16_t*)GR, ldgr, (const uint16_t*)GA, ldga,             \
                         (const uint16_t*)UP, ldup, (uint16_t*)DG, lddg, (uint16_t*)DU, lddu, \
                         (const uint16_t*)YG, (const uint16_t*)YU, ldy, M, K, kps, ws,        \
                         (uint16_t*)out, ldo, out_cols, alpha_g, alpha_u, (uint16_t*)out_t,   \
                         ldt);                                                                \
      hipLaunchKernelGGL((lora_down_reduce<IT, IT>), dim3(grid1d(M * out_cols)), dim3(256),   \
                         0, s, ws, splits, M, NC, (uint16_t*)out, ldo, out_cols, alpha_g,     \
                         alpha_u, (uint16_t*)out_t, ldt);                                     \
    }                                                                                         \
  } while (0)
  if (dtype == QL_BF16) QL_SWD(QL_BF16);
  else QL_SWD(QL_F16);
#undef QL_SWD
  return ql_launch_status();
}

// SwiGLU backward + both rank-16 products per adapter: one workgroup per 256 columns and
// row range, the ranges (multiples of 32 rows) chosen so the grid fills at most the two
// workgroups per CU that fit (more leaves a short second round).
int64_t ql_swiglu_bwd_lora_rows_per_split(int64_t M, int64_t K) {
  const int64_t blocks = (K + kSlCols - 1) / kSlCols;
  int64_t s = 512 / blocks;
  if (s < 1) s = 1;
  const int64_t rps = ((M + s - 1) / s + kSlRows - 1) / kSlRows * kSlRows;
  return rps > 0 ? rps : kSlRows;
}

int64_t ql_swiglu_bwd_lora_ws_floats(int64_t M, int64_t K, bool da) {
  const int64_t blocks = (K + kSlCols - 1) / kSlCols;
  const int64_t rps = ql_swiglu_bwd_lora_rows_per_split(M, K);
  const int64_t splits = (M + rps - 1) / rps;
  return blocks * M * 2 * kRank + (da ? 3 : 2) * splits * K * kRank;
}

int ql_swiglu_bwd_lora(int dtype, const void* GR, int64_t ldgr, const void* GA, int64_t ldga,
                       const void* UP, int64_t ldup, void* DG, int64_t lddg, void* DU,
                       int64_t lddu, int64_t M, int64_t K, const void* YG, const void* YU,
                       int64_t ldy, const void* UTG, const void* UTU, int64_t ldut,
                       float alpha_g, float alpha_u, float beta_g, float beta_u, void* out,
                       int64_t ldo, int out_cols, void* out_t, int64_t ldt, float* dbg,
                       float* dbu, const void* UTD, float beta_d, float* dad, float* ws,
                       int64_t ws_floats, hipStream_t s, const SwDrop* drop = nullptr) {
  constexpr int NC = 2 * kRank;
  const bool da = UTD != nullptr;
  if (drop && !da) return QL_EINVAL;
  const SwDrop dr = drop ? *drop : SwDrop{};
  if (M <= 0 || K <= 0 || K % 32 || out_cols < NC || ldo < out_cols) return QL_EINVAL;
  if (out_t && ldt < M) return QL_EINVAL;
  if (ldgr < K || ldga < K || ldup < K || lddg < K || lddu < K || ldy < K || ldut < M)
    return QL_EINVAL;
  // per-lane byte offsets within a tile's rows are 32-bit
  const int64_t lim = int64_t(1) << 31;
  if (2 * kSlRows * (ldgr > ldga ? (ldgr > ldup ? ldgr : ldup) : (ldga > ldup ? ldga : ldup)) >= lim ||
      2 * kSlRows * (lddg > lddu ? lddg : lddu) >= lim || 32 * ldy >= lim)
    return QL_EINVAL;
  if (!rows16_ok(GR, ldgr) || !rows16_ok(GA, ldga) || !rows16_ok(UP, ldup) ||
      !rows16_ok(DG, lddg) || !rows16_ok(DU, lddu) || !rows16_ok(YG, ldy) ||
      !rows16_ok(YU, ldy) || !rows16_ok(UTG, ldut) || !rows16_ok(UTU, ldut) ||
      (da && !rows16_ok(UTD, ldut)))
    return QL_EALIGN;
  if (!ql_aligned(dbg, 16) || !ql_aligned(dbu, 16) || !ql_aligned(ws, 16) ||
      (da && !ql_aligned(dad, 16)))
    return QL_EALIGN;
  if (dtype != QL_BF16 && dtype != QL_F16) return QL_EDTYPE;
  if (ws_floats < ql_swiglu_bwd_lora_ws_floats(M, K, da)) return QL_EINVAL;
  const int64_t blocks = (K + kSlCols - 1) / kSlCols;
  const int64_t rps = ql_swiglu_bwd_lora_rows_per_split(M, K);
  const int splits = (int)((M + rps - 1) / rps);
  if (blocks > INT32_MAX || splits > 65535) return QL_ESHAPE;
  float* ws_du = ws;
  float* ws_db = ws + blocks * M * NC;
  float* ws_da = ws_db + 2 * (int64_t)splits * K * kRank;
  const dim3 grid((unsigned)blocks, (unsigned)splits);
#define QL_SWL(IT)                                                                            \
  do {                                                                                        \
    if (da && drop)                                                                           \
      hipLaunchKernelGGL((swiglu_bwd_lora_kernel<IT, true, true>), grid, dim3(256), 0, s,     \
                         (const uint16_t*)GR, ldgr, (const uint16_t*)GA, ldga,                \
                         (const uint16_t*)UP, ldup, (uint16_t*)DG, lddg, (uint16_t*)DU,       \
                         lddu, (const uint16_t*)YG, (const uint16_t*)YU, ldy,                 \
                         (const uint16_t*)UTG, (const uint16_t*)UTU, ldut, M, K, rps, ws_du,  \
                         ws_db, (const uint16_t*)UTD, ws_da, dr);                             \
    else if (da)                                                                              \
      hipLaunchKernelGGL((swiglu_bwd_lora_kernel<IT, true, false>), grid, dim3(256), 0, s,    \
                         (const uint16_t*)GR, ldgr, (const uint16_t*)GA, ldga,                \
                         (const uint16_t*)UP, ldup, (uint16_t*)DG, lddg, (uint16_t*)DU,       \
                         lddu, (const uint16_t*)YG, (const uint16_t*)YU, ldy,                 \
                         (const uint16_t*)UTG, (const uint16_t*)UTU, ldut, M, K, rps, ws_du,  \
                         ws_db, (const uint16_t*)UTD, ws_da, dr);                             \
    else                                                                                      \
      hipLaunchKernelGGL((swiglu_bwd_lora_kernel<IT, false, false>), grid, dim3(256), 0, s,   \
                         (const uint16_t*)GR, ldgr, (const uint16_t*)GA, ldga,                \
                         (const uint16_t*)UP, ldup, (uint16_t*)DG, lddg, (uint16_t*)DU,       \
                         lddu, (const uint16_t*)YG, (const uint16_t*)YU, ldy,                 \
                         (const uint16_t*)UTG, (const uint16_t*)UTU, ldut, M, K, rps, ws_du,  \
                         ws_db, (const uint16_t*)nullptr, (float*)nullptr, dr);               \
    int st = ql_launch_status();                                                              \
    if (st != QL_OK) return st;                                                               \
    hipLaunchKernelGGL((lora_down_reduce<IT, IT>), dim3(grid1d(M * out_cols)), dim3(256), 0,  \
                       s, ws_du, (int)blocks, M, NC, (uint16_t*)out, ldo, out_cols, alpha_g,  \
                       alpha_u, (uint16_t*)out_t, ldt);                                       \
  } while (0)
  if (dtype == QL_BF16) QL_SWL(QL_BF16);
  else QL_SWL(QL_F16);
#undef QL_SWL
  int st = ql_launch_status();
  if (st != QL_OK) return st;
  // dB_gate, dB_up (and dA_down, [16, K]: A's layout) in one launch
  WgradReduceSet set{};
  set.ws[0] = ws_db;
  set.out[0] = dbg;
  set.alpha[0] = beta_g;
  set.ws[1] = ws_db + (int64_t)splits * K * kRank;
  set.out[1] = dbu;
  set.alpha[1] = beta_u;
  set.ws[2] = ws_da;
  set.out[2] = dad;
  set.alpha[2] = beta_d;
  set.out_t[2] = true;
  hipLaunchKernelGGL(lora_wgrad_reduce_set, dim3(grid64(K * kRank / 4), da ? 3 : 2), dim3(256),
                     0, s, set, splits, K, kRank);
  return ql_launch_status();
}

// SwiGLU forward + the down-projection of h: the backward_down tile walk and split rule.
int ql_swiglu_fwd_down(int dtype, const void* GA, int64_t ldga, const void* UP, int64_t ldup,
                       void* HH, int64_t ldh, int64_t M, int64_t K, const void* Y, int64_t ldy,
                       float alpha, void* out, int64_t ldo, int out_cols, void* out_t,
                       int64_t ldt, float* ws, int64_t ws_floats, hipStream_t s,
                       const SwDrop* drop = nullptr) {
  if (M <= 0 || K <= 0 || K % 32 || out_cols < kRank || ldo < out_cols) return QL_EINVAL;
  const SwDrop dr = drop ? *drop : SwDrop{};
  if (out_t && ldt < M) return QL_EINVAL;
  if (ldga < K || ldup < K || ldh < K || ldy < K) return QL_EINVAL;
  const int64_t lim = int64_t(1) << 31;
  if (2 * kSwRows * (ldga > ldup ? ldga : ldup) >= lim || 2 * kSwRows * ldh >= lim ||
      32 * ldy >= lim)
    return QL_EINVAL;
  if (!rows16_ok(GA, ldga) || !rows16_ok(UP, ldup) || !rows16_ok(HH, ldh) || !rows16_ok(Y, ldy))
    return QL_EALIGN;
  if (dtype != QL_BF16 && dtype != QL_F16) return QL_EDTYPE;
  int splits = ql_swiglu_fwd_down_splits(M, K, drop != nullptr);
  if (ws_floats < (int64_t)splits * M * kRank || !ws) splits = 1;
  int64_t kps = ((K + splits - 1) / splits + kSwK - 1) / kSwK * kSwK;
  splits = (int)((K + kps - 1) / kps);
  const dim3 grid((unsigned)((M + kSwRows - 1) / kSwRows), (unsigned)splits);
#define QL_SWF(IT)                  \
  do {                              \
    if (drop) QL_SWFD(IT, true);    \
    else QL_SWFD(IT, false);        \
  } while (0)
#define QL_SWFD(IT, DR)                                                                       \
  do {                                                                                        \
    if (splits == 1) {                                                                        \
      hipLaunchKernelGGL((swiglu_fwd_down_kernel<IT, false, DR>), grid, dim3(256), 0, s,      \
                         (const uint16_t*)GA, ldga, (const uint16_t*)UP, ldup, (uint16_t*)HH, \
                         ldh, (const uint16_t*)Y, ldy, M, K, kps, (float*)nullptr,            \
                         (uint16_t*)out, ldo, out_cols, alpha, (uint16_t*)out_t, ldt, dr);    \
    } else {                                                                                  \
      hipLaunchKernelGGL((swiglu_fwd_down_kernel<IT, true, DR>), grid, dim3(256), 0, s,       \
                         (const uint16_t*)GA, ldga, (const uint16_t*)UP, ldup, (uint16_t*)HH, \
                         ldh, (const uint16_t*)Y, ldy, M, K, kps, ws, (uint16_t*)out, ldo,    \
                         out_cols, alpha, (uint16_t*)out_t, ldt, dr);                         \
      hipLaunchKernelGGL((lora_down_reduce<IT, IT>), dim3(grid1d(M * out_cols)), dim3(256),   \
                         0, s, ws, splits, M, kRank, (uint16_t*)out, ldo, out_cols, alpha,    \
                         alpha, (uint16_t*)out_t, ldt);                                       \
    }                                                                                         \
  } while (0)
  if (dtype == QL_BF16) QL_SWF(QL_BF16);
  else QL_SWF(QL_F16);
#undef QL_SWF
#undef QL_SWFD
  return ql_launch_status();
}

// ---- C-ABI -------------------------------------------------------------------------------

extern "C" int64_t qlora_swiglu_bwd_lora_down_workspace_size(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const int s = ql_swiglu_bwd_down_splits(rows, cols);
  return s > 1 ? (int64_t)s * rows * 2 * kRank * (int64_t)sizeof(float) : 0;
}

extern "C" int qlora_swiglu_bwd_lora_down(
    const void* grad, int64_t ldgr, const void* gate, int64_t ldg, const void* up, int64_t ldu,
    void* dgate, int64_t lddg, void* dup, int64_t lddu, int64_t rows, int64_t cols,
    const void* bt_gate, const void* bt_up, int64_t ldbt, float alpha_gate, float alpha_up,
    int dtype, void* du, int64_t ldo, int out_cols, void* du_t, int64_t ldt, void* workspace,
    int64_t workspace_bytes, ql_stream_t stream) {
  if (rows < 0 || cols < 0 || workspace_bytes < 0) return QL_EINVAL;
  if (rows == 0) return QL_OK;
  if (!grad || !gate || !up || !dgate || !dup || !bt_gate || !bt_up || !du) return QL_EINVAL;
  // lanes past the last row or group recompute the last one and re-read its inputs after
  // other lanes stored: outputs that overlap the inputs would be read back modified
  const void* ins[3] = {grad, gate, up};
  const int64_t in_ld[3] = {ldgr, ldg, ldu};
  for (int i = 0; i < 3; ++i)
    if (ql_spans_overlap(dgate, lddg, ins[i], in_ld[i], rows, cols, 2) ||
        ql_spans_overlap(dup, lddu, ins[i], in_ld[i], rows, cols, 2))
      return QL_EINVAL;
  if (workspace && !ql_aligned(workspace, 16)) return QL_EALIGN;
  if (!ql_aligned(du, 2) || (du_t && !ql_aligned(du_t, 2))) return QL_EALIGN;
  return ql_swiglu_bwd_down(dtype, grad, ldgr, gate, ldg, up, ldu, dgate, lddg, dup, lddu, rows,
                            cols, bt_gate, bt_up, ldbt, alpha_gate, alpha_up, du, ldo, out_cols,
                            du_t, ldt, static_cast<float*>(workspace),
                            workspace_bytes / (int64_t)sizeof(float),
                            static_cast<hipStream_t>(stream));
}


// The dropout arguments of the two entries below: 0 < p < 1, bits 8-B aligned, group stride a
// multiple of 8 and >= cols.
static int swiglu_drop_args(uint64_t seed, float p, float scale, void* bits, int64_t gs,
                            int64_t cols, bool draw, SwDrop* out) {
  if (!(p > 0.0f) || !(p < 1.0f) || !bits) return QL_EINVAL;
  if (!ql_aligned(bits, 8)) return QL_EALIGN;
  if (gs < cols || gs % 8) return QL_ESHAPE;
  out->seed = seed;
  out->thr = draw ? ql_philox::keep_threshold(p) : 0u;
  out->scale = scale;
  out->bits = static_cast<uint8_t*>(bits);
  out->gs = gs;
  return QL_OK;
}

extern "C" int qlora_swiglu_fwd_lora_down_dropout(
    const void* gate, int64_t ldg, const void* up, int64_t ldu, void* h, int64_t ldh,
    int64_t rows, int64_t cols, const void* a, int64_t lda, float alpha, int dtype, void* u,
    int64_t ldo, int out_cols, void* u_t, int64_t ldt, uint64_t seed, float p, float scale,
    uint8_t* bits, int64_t bits_group_stride, void* workspace, int64_t workspace_bytes,
    ql_stream_t stream) {
  if (rows < 0 || cols < 0 || workspace_bytes < 0) return QL_EINVAL;
  SwDrop dr{};
  const int st = swiglu_drop_args(seed, p, scale, bits, bits_group_stride, cols, true, &dr);
  if (st != QL_OK) return st;
  if (rows == 0) return QL_OK;
  if (!gate || !up || !h || !a || !u) return QL_EINVAL;
  if (ql_spans_overlap(h, ldh, gate, ldg, rows, cols, 2) ||
      ql_spans_overlap(h, ldh, up, ldu, rows, cols, 2))
    return QL_EINVAL;
  if (workspace && !ql_aligned(workspace, 16)) return QL_EALIGN;
  if (!ql_aligned(u, 2) || (u_t && !ql_aligned(u_t, 2))) return QL_EALIGN;
  return ql_swiglu_fwd_down(dtype, gate, ldg, up, ldu, h, ldh, rows, cols, a, lda, alpha, u, ldo,
                            out_cols, u_t, ldt, static_cast<float*>(workspace),
                            workspace_bytes / (int64_t)sizeof(float),
                            static_cast<hipStream_t>(stream), &dr);
}

extern "C" int qlora_swiglu_bwd_lora_dropout(
    const void* grad, int64_t ldgr, const void* gate, int64_t ldg, const void* up, int64_t ldu,
    void* dgate, int64_t lddg, void* dup, int64_t lddu, int64_t rows, int64_t cols,
    const void* bt_gate, const void* bt_up, int64_t ldbt, const void* ut_gate,
    const void* ut_up, int64_t ldut, float alpha_gate, float alpha_up, float beta_gate,
    float beta_up, int dtype, void* du, int64_t ldo, int out_cols, void* du_t, int64_t ldt,
    float* db_gate, float* db_up, const void* ud_t, float beta_down, float* da_down,
    const uint8_t* bits, int64_t bits_group_stride, float p, float scale, const void* du_add,
    int64_t ld_du_add, const void* a_add, int64_t ld_a_add, void* workspace,
    int64_t workspace_bytes, ql_stream_t stream) {
  if (rows < 0 || cols < 0 || workspace_bytes < 0) return QL_EINVAL;
  SwDrop dr{};
  int st = swiglu_drop_args(0, p, scale, const_cast<uint8_t*>(bits), bits_group_stride, cols,
                            false, &dr);
  if (st != QL_OK) return st;
  if (du_add) {
    if (!a_add || ld_du_add < kRank || ld_a_add < cols) return QL_EINVAL;
    if (!ql_aligned(du_add, 8) || ld_du_add % 4) return QL_EALIGN;
    dr.add_du = static_cast<const uint16_t*>(du_add);
    dr.add_ldu = ld_du_add;
    dr.add_a = static_cast<const uint16_t*>(a_add);
    dr.add_lda = ld_a_add;
  }
  if (rows == 0) return QL_OK;
  if (!grad || !gate || !up || !dgate || !dup || !bt_gate || !bt_up || !ut_gate || !ut_up ||
      !du || !db_gate || !db_up || !workspace || !ud_t || !da_down)
    return QL_EINVAL;
  const void* ins[3] = {grad, gate, up};
  const int64_t in_ld[3] = {ldgr, ldg, ldu};
  for (int i = 0; i < 3; ++i)
    if (ql_spans_overlap(dgate, lddg, ins[i], in_ld[i], rows, cols, 2) ||
        ql_spans_overlap(dup, lddu, ins[i], in_ld[i], rows, cols, 2))
      return QL_EINVAL;
  if (!ql_aligned(du, 2) || (du_t && !ql_aligned(du_t, 2))) return QL_EALIGN;
  return ql_swiglu_bwd_lora(dtype, grad, ldgr, gate, ldg, up, ldu, dgate, lddg, dup, lddu, rows,
                            cols, bt_gate, bt_up, ldbt, ut_gate, ut_up, ldut, alpha_gate,
                            alpha_up, beta_gate, beta_up, du, ldo, out_cols, du_t, ldt, db_gate,
                            db_up, ud_t, beta_down, da_down, static_cast<float*>(workspace),
                            workspace_bytes / (int64_t)sizeof(float),
                            static_cast<hipStream_t>(stream), &dr);
}

extern "C" int64_t qlora_swiglu_bwd_lora_workspace_size(int64_t rows, int64_t cols,
                                                        int with_da) {
  if (rows <= 0 || cols <= 0 || cols % 32) return 0;
  return ql_swiglu_bwd_lora_ws_floats(rows, cols, with_da != 0) * (int64_t)sizeof(float);
}

extern "C" int qlora_swiglu_bwd_lora(
    const void* grad, int64_t ldgr, const void* gate, int64_t ldg, const void* up, int64_t ldu,
    void* dgate, int64_t lddg, void* dup, int64_t lddu, int64_t rows, int64_t cols,
    const void* bt_gate, const void* bt_up, int64_t ldbt, const void* ut_gate,
    const void* ut_up, int64_t ldut, float alpha_gate, float alpha_up, float beta_gate,
    float beta_up, int dtype, void* du, int64_t ldo, int out_cols, void* du_t, int64_t ldt,
    float* db_gate, float* db_up, const void* ud_t, float beta_down, float* da_down,
    void* workspace, int64_t workspace_bytes, ql_stream_t stream) {
  if (rows < 0 || cols < 0 || workspace_bytes < 0) return QL_EINVAL;
  if (rows == 0) return QL_OK;
  if (!grad || !gate || !up || !dgate || !dup || !bt_gate || !bt_up || !ut_gate || !ut_up ||
      !du || !db_gate || !db_up || !workspace || (!ud_t) != (!da_down))
    return QL_EINVAL;
  // lanes past the last row or column recompute the last one and re-read its inputs after
  // other lanes stored: outputs that overlap the inputs would be read back modified
  const void* ins[3] = {grad, gate, up};
  const int64_t in_ld[3] = {ldgr, ldg, ldu};
  for (int i = 0; i < 3; ++i)
    if (ql_spans_overlap(dgate, lddg, ins[i], in_ld[i], rows, cols, 2) ||
        ql_spans_overlap(dup, lddu, ins[i], in_ld[i], rows, cols, 2))
      return QL_EINVAL;
  if (!ql_aligned(du, 2) || (du_t && !ql_aligned(du_t, 2))) return QL_EALIGN;
  return ql_swiglu_bwd_lora(dtype, grad, ldgr, gate, ldg, up, ldu, dgate, lddg, dup, lddu, rows,
                            cols, bt_gate, bt_up, ldbt, ut_gate, ut_up, ldut, alpha_gate,
                            alpha_up, beta_gate, beta_up, du, ldo, out_cols, du_t, ldt, db_gate,
                            db_up, ud_t, beta_down, da_down, static_cast<float*>(workspace),
                            workspace_bytes / (int64_t)sizeof(float),
                            static_cast<hipStream_t>(stream));
}

extern "C" int64_t qlora_swiglu_fwd_lora_down_workspace_size(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  // enough for either form (the dropout form splits further)
  const int s0 = ql_swiglu_fwd_down_splits(rows, cols, false);
  const int s1 = ql_swiglu_fwd_down_splits(rows, cols, true);
  const int s = s0 > s1 ? s0 : s1;
  return s > 1 ? (int64_t)s * rows * kRank * (int64_t)sizeof(float) : 0;
}

extern "C" int qlora_swiglu_fwd_lora_down(const void* gate, int64_t ldg, const void* up,
                                          int64_t ldu, void* h, int64_t ldh, int64_t rows,
                                          int64_t cols, const void* a, int64_t lda, float alpha,
                                          int dtype, void* u, int64_t ldo, int out_cols,
                                          void* u_t, int64_t ldt, void* workspace,
                                          int64_t workspace_bytes, ql_stream_t stream) {
  if (rows < 0 || cols < 0 || workspace_bytes < 0) return QL_EINVAL;
  if (rows == 0) return QL_OK;
  if (!gate || !up || !h || !a || !u) return QL_EINVAL;
  // lanes past the last row or column recompute the last one and re-read its inputs after
  // other lanes stored: an output that overlaps the inputs would be read back modified
  if (ql_spans_overlap(h, ldh, gate, ldg, rows, cols, 2) ||
      ql_spans_overlap(h, ldh, up, ldu, rows, cols, 2))
    return QL_EINVAL;
  if (workspace && !ql_aligned(workspace, 16)) return QL_EALIGN;
  if (!ql_aligned(u, 2) || (u_t && !ql_aligned(u_t, 2))) return QL_EALIGN;
  return ql_swiglu_fwd_down(dtype, gate, ldg, up, ldu, h, ldh, rows, cols, a, lda, alpha, u, ldo,
                            out_cols, u_t, ldt, static_cast<float*>(workspace),
                            workspace_bytes / (int64_t)sizeof(float),
                            static_cast<hipStream_t>(stream));
}

extern "C" int64_t qlora_lora_down_workspace_size(int64_t M, int64_t K, int slots) {
  if (M <= 0 || K <= 0 || slots < 1 || slots > kMaxSlots) return 0;
  return ql_lora_down_workspace_floats(M, K, slots) * (int64_t)sizeof(float);
}

extern "C" int qlora_lora_down(const void* X, int64_t ldx, const void* Y, int64_t ldy, int64_t M,
                               int64_t K, int slots, int in_dtype, void* out, int64_t ldo,
                               int out_cols, int out_dtype, float alpha, void* out_t, int64_t ldt,
                               void* workspace, int64_t workspace_bytes, ql_stream_t stream) {
  if (M < 0 || K < 0 || workspace_bytes < 0) return QL_EINVAL;
  if (M == 0) return QL_OK;
  if (!X || !Y || !out) return QL_EINVAL;
  if (workspace && !ql_aligned(workspace, 16)) return QL_EALIGN;
  if (out_t && !ql_aligned(out_t, 2)) return QL_EALIGN;
  return ql_lora_down(in_dtype, out_dtype, X, ldx, Y, ldy, M, K, slots, out, ldo, out_cols,
                      alpha, out_t, ldt, static_cast<float*>(workspace),
                      workspace_bytes / (int64_t)sizeof(float),
                      static_cast<hipStream_t>(stream));
}

// K split of the fused dropout + down-projection: up to 1024 workgroups of 8 waves, keeping at
// least four chunks per wave in every split. Measured at 4096 rows (bf16, one adapter): K =
// 18944 126-128 us split 4 against 135-136 us unsplit; at K = 3584 the split (then 4 x 14
// chunks) cost 4-24 us more than it saved (the partials and their reduce), so it stays unsplit.
static int ql_dropout_down_splits(int64_t M, int64_t K) {
  const int64_t blocks = (M + 15) / 16, nch = K / 64;
  int s = 1;
  while (blocks * s < 1024 && nch / (2 * s) >= 4 * kDdWaves && s < 64) s *= 2;
  return s;
}

static int64_t ql_dropout_down_workspace_bytes(int64_t M, int64_t K, int slots) {
  const int s = ql_dropout_down_splits(M, K);
  return s > 1 ? (int64_t)s * M * kRank * slots * (int64_t)sizeof(float) : 0;
}

extern "C" int64_t qlora_lora_dropout_down_workspace_size(int64_t M, int64_t K, int slots) {
  if (M <= 0 || K <= 0 || K % 64 || slots < 1 || slots > kMaxSlots) return 0;
  return ql_dropout_down_workspace_bytes(M, K, slots);
}

extern "C" int qlora_lora_dropout_down(const void* x, int64_t x_row_stride, const void* A,
                                       int64_t a_row_stride, int64_t M, int64_t K, int slots,
                                       int dtype, const uint64_t* seeds, float p, float scale,
                                       void* const* xd, int64_t xd_row_stride,
                                       uint8_t* const* bits, int64_t bits_group_stride, void* u,
                                       int64_t u_row_stride, int u_cols, void* u_t,
                                       int64_t u_t_row_stride, void* workspace,
                                       int64_t workspace_bytes, ql_stream_t stream) {
  if (M < 0 || K < 0 || slots < 1 || slots > kMaxSlots || !(p > 0.0f) || !(p < 1.0f) ||
      workspace_bytes < 0)
    return QL_EINVAL;
  if (dtype != QL_BF16 && dtype != QL_F16) return QL_EDTYPE;
  if (M == 0 || K == 0) return QL_OK;
  if (!x || !A || !seeds || !bits || !u) return QL_EINVAL;
  if (workspace && !ql_aligned(workspace, 16)) return QL_EALIGN;
  DropDownSlots sl{};
  for (int g = 0; g < slots; ++g) {
    if ((xd && !xd[g]) || !bits[g]) return QL_EINVAL;
    if (xd && !ql_aligned(xd[g], 16)) return QL_EALIGN;
    sl.seed[g] = seeds[g];
    sl.xd[g] = xd ? static_cast<uint16_t*>(xd[g]) : nullptr;
    sl.bits[g] = bits[g];
  }
  const int nc = kRank * slots;
  if (K % 64 || x_row_stride < K || a_row_stride < K || (xd && xd_row_stride < K) ||
      bits_group_stride < K || bits_group_stride % 8 || u_cols < nc || u_row_stride < u_cols ||
      (u_t && u_t_row_stride < M))
    return QL_ESHAPE;
  if (x_row_stride % 8 || a_row_stride % 8 || (xd && xd_row_stride % 8) || !ql_aligned(x, 16) ||
      !ql_aligned(A, 16) || !ql_aligned(u, 2) || (u_t && !ql_aligned(u_t, 2)))
    return QL_EALIGN;
  const int64_t gx = (M + 15) / 16;
  if (gx > INT32_MAX) return QL_ESHAPE;
  int splits = ql_dropout_down_splits(M, K);
  if (workspace_bytes < ql_dropout_down_workspace_bytes(M, K, slots) || !workspace) splits = 1;
  const int64_t nch = K / 64;
  const int64_t cps = (nch + splits - 1) / splits;
  splits = (int)((nch + cps - 1) / cps);
  const uint32_t thr = ql_philox::keep_threshold(p);
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* ws = static_cast<float*>(workspace);
  const dim3 grid((unsigned)gx, (unsigned)splits);
#define QL_DD(DT, G)                \
  do {                              \
    if (xd) QL_DDX(DT, G, true);    \
    else QL_DDX(DT, G, false);      \
  } while (0)
#define QL_DDX(DT, G, XD)                                                                     \
  do {                                                                                        \
    if (splits == 1) {                                                                        \
      hipLaunchKernelGGL((dropout_down_kernel<DT, G, false, XD>), grid, dim3(64 * kDdWaves), 0, s, \
                         (const uint16_t*)x, x_row_stride, (const uint16_t*)A, a_row_stride,  \
                         M, K, cps, sl, xd_row_stride, bits_group_stride, thr, scale,           \
                         (float*)nullptr, (uint16_t*)u, u_row_stride, u_cols,                 \
                         (uint16_t*)u_t, u_t_row_stride);                                     \
    } else {                                                                                  \
      hipLaunchKernelGGL((dropout_down_kernel<DT, G, true, XD>), grid, dim3(64 * kDdWaves), 0, s, \
                         (const uint16_t*)x, x_row_stride, (const uint16_t*)A, a_row_stride,  \
                         M, K, cps, sl, xd_row_stride, bits_group_stride, thr, scale, ws,       \
                         (uint16_t*)u, u_row_stride, u_cols, (uint16_t*)u_t, u_t_row_stride); \
      hipLaunchKernelGGL((lora_down_reduce<DT, DT>), dim3(grid1d(M * u_cols)), dim3(256), 0,   \
                         s, ws, splits, M, nc, (typename Elem<DT>::T*)u, u_row_stride, u_cols, \
                         1.0f, 1.0f, (uint16_t*)u_t, u_t_row_stride);                         \
    }                                                                                         \
  } while (0)
#define QL_DD_G(DT)                \
  switch (slots) {                 \
    case 1: QL_DD(DT, 1); break;   \
    case 2: QL_DD(DT, 2); break;   \
    case 3: QL_DD(DT, 3); break;   \
    default: QL_DD(DT, 4); break;  \
  }
  if (dtype == QL_BF16) {
    QL_DD_G(QL_BF16)
  } else {
    QL_DD_G(QL_F16)
  }
#undef QL_DD_G
#undef QL_DD
#undef QL_DDX
  return ql_launch_status();
}

extern "C" int64_t qlora_lora_wgrad_workspace_size(int64_t M, int64_t N, int slots) {
  if (M <= 0 || N <= 0 || slots < 1 || slots > kMaxSlots) return 0;
  return ql_lora_wgrad_workspace_floats(M, N, slots) * (int64_t)sizeof(float);
}

extern "C" int qlora_lora_wgrad(const void* PT, int64_t ldpt, const void* Q, int64_t ldq, int64_t M,
                                int64_t N, int slots, int in_dtype, float* out,
                                int out_transposed, float alpha, void* workspace,
                                int64_t workspace_bytes, ql_stream_t stream) {
  if (M < 0 || N < 0 || workspace_bytes < 0 || slots < 1 || slots > kMaxSlots) return QL_EINVAL;
  if (N == 0) return QL_OK;
  if (!PT || !Q || !out) return QL_EINVAL;
  if (M == 0) {  // an empty reduction: zeros (a fill kernel, not a memset node)
    if (!ql_aligned(out, 16)) return QL_EALIGN;
    hipLaunchKernelGGL(lora_wgrad_reduce, dim3(grid64(N * kRank * slots / 4)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), (const float*)nullptr, 0, N,
                       kRank * slots, out, 0.f, out_transposed != 0);
    return ql_launch_status();
  }
  if (workspace && !ql_aligned(workspace, 16)) return QL_EALIGN;
  return ql_lora_wgrad(in_dtype, PT, ldpt, Q, ldq, M, N, slots, out, out_transposed, alpha,
                       static_cast<float*>(workspace), workspace_bytes / (int64_t)sizeof(float),
                       static_cast<hipStream_t>(stream));
}

// Weight gradients of several adapters whose outputs are concatenated, as one multi-slot
// pass over the concatenated output gradient (every slot's products over every column, the
// unused ones discarded by lora_wgrad_reduce_diag): one read of Q and two launches instead of
// two per adapter.
static int64_t wgrad_diag_floats(int64_t M, int64_t N, int slots) {
  return (int64_t)ql_lora_wgrad_splits(M, N, slots) * N * kRank * slots;
}

extern "C" int qlora_lora_wgrad_masked(const void* PT, int64_t ldpt, const void* Q, int64_t ldq,
                                       int64_t M, int64_t N, int slots, int in_dtype,
                                       const uint8_t* const* bits, int64_t bits_group_stride,
                                       float scale, float* out, float alpha, void* workspace,
                                       int64_t workspace_bytes, ql_stream_t stream) {
  if (M < 0 || N < 0 || workspace_bytes < 0 || slots < 1 || slots > kMaxSlots) return QL_EINVAL;
  if (N == 0) return QL_OK;
  if (!PT || !Q || !out || !bits) return QL_EINVAL;
  WgradMask mk{};
  for (int g = 0; g < slots; ++g) {
    if (!bits[g]) return QL_EINVAL;
    if (!ql_aligned(bits[g], 8)) return QL_EALIGN;
    mk.p[g] = bits[g];
  }
  if (N % 8 || bits_group_stride < N || bits_group_stride % 8) return QL_ESHAPE;
  mk.gs = bits_group_stride;
  mk.scale = scale;
  if (M == 0) {  // an empty reduction: zeros (a fill kernel, not a memset node)
    if (!ql_aligned(out, 16)) return QL_EALIGN;
    hipLaunchKernelGGL(lora_wgrad_reduce, dim3(grid64(N * kRank * slots / 4)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), (const float*)nullptr, 0, N,
                       kRank * slots, out, 0.f, true);
    return ql_launch_status();
  }
  if (workspace && !ql_aligned(workspace, 16)) return QL_EALIGN;
  return ql_lora_wgrad(in_dtype, PT, ldpt, Q, ldq, M, N, slots, out, 1, alpha,
                       static_cast<float*>(workspace), workspace_bytes / (int64_t)sizeof(float),
                       static_cast<hipStream_t>(stream), &mk);
}

extern "C" int64_t qlora_lora_wgrad_diag_workspace_size(int64_t M, int64_t N, int slots) {
  if (M <= 0 || N <= 0 || slots < 1 || slots > kMaxSlots) return 0;
  return wgrad_diag_floats(M, N, slots) * (int64_t)sizeof(float);
}

extern "C" int qlora_lora_wgrad_diag(const void* PT, int64_t ldpt, const void* Q, int64_t ldq,
                                     int64_t M, int64_t N, int slots, int in_dtype,
                                     const int64_t* col_offsets, const float* alphas,
                                     float* out, void* workspace, int64_t workspace_bytes,
                                     ql_stream_t stream) {
  if (M <= 0 || N < 0 || slots < 1 || slots > kMaxSlots) return QL_EINVAL;
  if (N == 0) return QL_OK;
  if (!PT || !Q || !out || !col_offsets || !alphas || !workspace) return QL_EINVAL;
  WgradDiag d{};
  d.slots = slots;
  for (int q = 0; q <= slots; ++q) d.off[q] = col_offsets[q];
  if (d.off[0] != 0 || d.off[slots] != N) return QL_ESHAPE;
  for (int q = 0; q < slots; ++q) {
    if (d.off[q + 1] < d.off[q]) return QL_ESHAPE;
    d.alpha[q] = alphas[q];
  }
  const int nc = kRank * slots;
  if (N % 8 || ldpt < M || ldq < N) return QL_EINVAL;
  if (64 * ldq >= (int64_t(1) << 31) || 2 * nc * ldpt >= (int64_t(1) << 31)) return QL_EINVAL;
  if (ldq % 8 || ldpt % 8 || !ql_aligned(Q, 16) || !ql_aligned(PT, 16) || !ql_aligned(out, 16) ||
      !ql_aligned(workspace, 16))
    return QL_EALIGN;
  if (in_dtype != QL_BF16 && in_dtype != QL_F16) return QL_EDTYPE;
  if (workspace_bytes < wgrad_diag_floats(M, N, slots) * (int64_t)sizeof(float)) return QL_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* ws = static_cast<float*>(workspace);
  int splits = ql_lora_wgrad_splits(M, N, slots);
  const int64_t mps = ((M + splits - 1) / splits + 127) / 128 * 128;
  splits = (int)((M + mps - 1) / mps);
  const dim3 grid((unsigned)((N + 127) / 128), (unsigned)splits);
  const int64_t per_wave = mps / 128;
  const int unroll = (slots == 1 && per_wave % 4 == 0) ? 4 : (per_wave % 2 == 0 ? 2 : 1);
#define QL_WD_GU(IT, G, U)                                                                     \
  hipLaunchKernelGGL((lora_wgrad_kernel<IT, true, G, U, false>), grid, dim3(kThreads), 0, s,   \
                     (const uint16_t*)PT, ldpt, (const uint16_t*)Q, ldq, M, N, mps, ws,         \
                     (float*)nullptr, 0.f, false, WgradMask{})
#define QL_WD_G(IT, G)                                     \
  do {                                                     \
    if (unroll == 4) QL_WD_GU(IT, G, (G == 1 ? 4 : 2));    \
    else if (unroll == 2) QL_WD_GU(IT, G, 2);              \
    else QL_WD_GU(IT, G, 1);                               \
  } while (0)
#define QL_WD(IT)                            \
  do {                                       \
    switch (slots) {                         \
      case 1: QL_WD_G(IT, 1); break;         \
      case 2: QL_WD_G(IT, 2); break;         \
      case 3: QL_WD_G(IT, 3); break;         \
      default: QL_WD_G(IT, 4); break;        \
    }                                        \
  } while (0)
  if (in_dtype == QL_BF16) QL_WD(QL_BF16);
  else QL_WD(QL_F16);
#undef QL_WD
#undef QL_WD_G
#undef QL_WD_GU
  hipLaunchKernelGGL(lora_wgrad_reduce_diag, dim3(grid1d(N * kRank / 4)), dim3(256), 0, s, ws,
                     splits, N, d, out);
  return ql_launch_status();
}

// ---- qlora_lora_wgrad without a caller workspace -------------------------------------------
// The split partials live in a file-scope device array instead: each GPU the library runs on
// holds its own kWgradScratchBytes copy until the process ends. On the host the array's name
// is a stand-in, not a device address, so host code never passes it to a kernel: it uses the
// address hipGetSymbolAddress returns, looked up once per device with that device current and
// kept per device. Every call on a GPU reuses that GPU's array; each split writes its whole
// partial before the reduce reads it, so nothing needs clearing, and calls that overlap on one
// GPU (two streams, two threads) race on it.
constexpr int64_t kWgradScratchBytes = int64_t(16) << 20;
static __device__ __align__(256) float lora_wgrad_scratch[kWgradScratchBytes / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices];  // device address of lora_wgrad_scratch per device, or null

// The device the launch goes to: the stream's, or the current one for the null stream.
int wgrad_scratch_of(hipStream_t stream, float** out) {
  int dev = 0;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return ql_hip_status(e);
  if (dev < 0 || dev >= kMaxDevices) return QL_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    int cur = 0;
    if ((e = hipGetDevice(&cur)) != hipSuccess) return ql_hip_status(e);
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return ql_hip_status(e);
    void* p = nullptr;
    const hipError_t got = hipGetSymbolAddress(&p, HIP_SYMBOL(lora_wgrad_scratch));
    if (cur != dev && (e = hipSetDevice(cur)) != hipSuccess) return ql_hip_status(e);
    if (got != hipSuccess) return ql_hip_status(got);
    if (!p || !ql_aligned(p, 256)) return QL_EALIGN;
    g_scratch[dev] = static_cast<float*>(p);
  }
  *out = g_scratch[dev];
  return QL_OK;
}

}  // namespace

extern "C" int qlora_lora_wgrad_noalloc(const void* PT, int64_t ldpt, const void* Q, int64_t ldq,
                                        int64_t M, int64_t N, int slots, int in_dtype, float* out,
                                        int out_transposed, float alpha, ql_stream_t stream) {
  if (M < 0 || N < 0 || slots < 1 || slots > kMaxSlots) return QL_EINVAL;
  if (N == 0) return QL_OK;
  if (!PT || !Q || !out) return QL_EINVAL;
  const int64_t need = M > 0 ? ql_lora_wgrad_workspace_floats(M, N, slots) * (int64_t)sizeof(float)
                             : 0;
  if (need > kWgradScratchBytes) return QL_ESHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (need == 0)  // unsplit (or empty) reductions use no scratch: the workspace entry point as is
    return qlora_lora_wgrad(PT, ldpt, Q, ldq, M, N, slots, in_dtype, out, out_transposed, alpha,
                            nullptr, 0, stream);
  float* ws = nullptr;
  const int st = wgrad_scratch_of(s, &ws);
  if (st != QL_OK) return st;
  return qlora_lora_wgrad(PT, ldpt, Q, ldq, M, N, slots, in_dtype, out, out_transposed, alpha, ws,
                          need, stream);
}

namespace {
// pad % 8 == 0, pad >= 16 G, K % 8 == 0, at and bs 16-B aligned (checked by the callers)
int launch_pack_group(const PackGroupArgs& p, int64_t K, int out_dtype, void* a16, void* at_pad,
                      void* bs_pad, void* bt, int pad, hipStream_t s) {
  const int64_t N = p.off[p.G];
  const int64_t total = (K + N) * (pad / 8) + N + (int64_t)kRank * p.G * K / 8;
  if (total == 0) return QL_OK;
  if (out_dtype == QL_BF16)
    hipLaunchKernelGGL((lora_pack_group_kernel<QL_BF16>), dim3(grid1d(total)), dim3(256), 0, s, p,
                       K, (uint16_t*)a16, (uint16_t*)at_pad, (uint16_t*)bs_pad, (uint16_t*)bt, pad);
  else
    hipLaunchKernelGGL((lora_pack_group_kernel<QL_F16>), dim3(grid1d(total)), dim3(256), 0, s, p,
                       K, (uint16_t*)a16, (uint16_t*)at_pad, (uint16_t*)bs_pad, (uint16_t*)bt, pad);
  return ql_launch_status();
}
}  // namespace

extern "C" int qlora_lora_pack(const float* A, const float* B, int64_t K, int64_t N, float scaling,
                               int out_dtype, void* a16, void* at_pad, void* bs_pad, void* bt,
                               int pad, ql_stream_t stream) {
  if (K < 0 || N < 0 || pad < kRank || K % 8) return QL_EINVAL;
  if (K == 0 && N == 0) return QL_OK;
  if (!A || !B || !a16 || !at_pad || !bs_pad || !bt) return QL_EINVAL;
  if (out_dtype != QL_BF16 && out_dtype != QL_F16) return QL_EDTYPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (pad % 8 == 0 && ql_aligned(at_pad, 16) && ql_aligned(bs_pad, 16)) {
    // the one-slot case of the group packing: the same values, 16-B chunks per item
    PackGroupArgs p{};
    p.G = 1;
    p.A[0] = A;
    p.B[0] = B;
    p.scale[0] = scaling;
    p.off[0] = 0;
    p.off[1] = N;
    return launch_pack_group(p, K, out_dtype, a16, at_pad, bs_pad, bt, pad, s);
  }
  const int64_t total = K + N + kRank * K / 8;
  const dim3 grid(grid1d(total));
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
  return launch_pack_group(p, K, out_dtype, a16, at_pad, bs_pad, bt, pad,
                           static_cast<hipStream_t>(stream));
}

extern "C" int qlora_lora_pack_jobs(const ql_lora_pack_job* jobs, int njobs, int64_t max_items,
                                    void* out_base, int out_dtype, int pad, ql_stream_t stream) {
  if (njobs < 0 || njobs > 65535 || max_items < 0 || pad < kRank || pad % 8) return QL_EINVAL;
  if (njobs == 0 || max_items == 0) return QL_OK;
  if (!jobs || !out_base) return QL_EINVAL;
  if (!ql_aligned(out_base, 16)) return QL_EALIGN;
  if (out_dtype != QL_BF16 && out_dtype != QL_F16) return QL_EDTYPE;
  // about 8 items a thread for the largest job, at most 256 workgroups a job
  int64_t gx = (max_items + 256 * 8 - 1) / (256 * 8);
  gx = gx < 1 ? 1 : (gx > 256 ? 256 : gx);
  const dim3 grid((unsigned)gx, (unsigned)njobs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (out_dtype == QL_BF16)
    hipLaunchKernelGGL((lora_pack_jobs_kernel<QL_BF16>), grid, dim3(256), 0, s, jobs,
                       (char*)out_base, pad);
  else
    hipLaunchKernelGGL((lora_pack_jobs_kernel<QL_F16>), grid, dim3(256), 0, s, jobs,
                       (char*)out_base, pad);
  return ql_launch_status();
}
