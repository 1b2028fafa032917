// Large-tile NT GEMM on CDNA4 matrix cores, with optional split-K:
//
//   C[M,N] = alpha * sum_k A[m,k] * B[n,k]  (+ beta * C) (+ bias[n])
//
// A [M,K] and B [N,K] are k-contiguous 16-bit matrices (bf16 or fp16), fp32 accumulation.
// This is the shape of every large contraction of the QLoRA step once weights are laid out
// k-contiguous: x @ W^T (solution/nf4.py:102), dY @ W with W dequantised transposed
// (solution/nf4.py:111), the lm_head chunk GEMM (solution/cross_entropy.py:117) and
// dz @ W with the head weight transposed (solution/cross_entropy.py:123).
//
// Tiling for gfx950 (256 CUs in 8 XCDs, wave64, 160 KiB LDS per CU, 512 VGPRs per lane):
//   - workgroup tile 256 x 256 x 64, 256 threads = 4 waves in a 2 x 2 grid; each wave owns a
//     128 x 128 block of C as 8 x 8 v_mfma_f32_16x16x32 accumulators (256 fp32 per lane, held
//     in AGPRs), so every 16-B fragment read from LDS feeds 8 MFMAs;
//   - operands go global -> LDS with global_load_lds_dwordx4 (no VGPR staging, no ds_write):
//     each wave instruction fills 1 KiB of LDS = 8 rows of 64 k. Rows are 128 B with the
//     16-B chunks XOR-swizzled by (row & 7), so both the DMA writes and the fragment reads
//     (ds_read_b128, 8 rows x 16 B per phase) hit all 32 banks once;
//   - two LDS stages (2 x 64 KiB), software-pipelined across K steps: each step multiplies
//     the first 32-k half of its stage while reading the second half's fragments, meets the
//     other waves at the one barrier of the step, starts the DMA of step k+2 into the stage
//     just consumed, and multiplies the second half while reading the first-half fragments
//     of step k+1 (scheduling barriers keep that instruction order). Fragment reads are
//     never exposed at a step boundary and the DMA has a full step to land;
//   - workgroup ids are remapped so that the tiles one XCD runs at a time are neighbours
//     (XCDs take workgroups round-robin; each has its own L2), then rastered in groups of 4
//     tile rows so that concurrently running tiles share A and B panels in L2;
//   - a second K segment C += A2 B2^T (K2 % 64 == 0, same M and N) can follow the first:
//     the rank-16 LoRA term of a LoRA linear rides along as one extra K step of the base
//     GEMM (x W^T + u (sB)^T with u, sB zero-padded to 64 columns) instead of separate
//     skinny GEMMs and an elementwise add;
//   - split-K: blockIdx.y selects a K range; each split writes an fp32 partial tile to a
//     caller-provided workspace and `splitk_reduce` sums the partials in split order
//     (deterministic) and applies alpha / beta / bias / the output type.
// Requirements (checked by the host): K % 64 == 0, lda % 8 == 0, ldb % 8 == 0, A and B
// 16-B aligned. M and N may be anything: edge rows are loaded clamped and never stored.
#include "ql_vec.h"
#include "gemm_nt.h"

namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) void* gbl_ptr_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

constexpr int BM = 256, BK = 64;
// Tile width: NJ 16-column fragments per wave, 2 waves across N (NJ = 8: 256; NJ = 7: 224).
template <int NJ> constexpr int bn_of() { return 32 * NJ; }
constexpr int kThreads = 256;
constexpr int kRowBytes = BK * 2;                  // 128 B: one tile row of 64 k
constexpr int kTileBytes = 256 * kRowBytes;        // 32 KiB: one operand, one stage
constexpr int kStageBytes = 2 * kTileBytes;        // A + B
constexpr int kGroupM = 4;

template <int DT> QL_DEV f32x4_t mfma(const uint4& a, const uint4& b, f32x4_t c);
template <> QL_DEV f32x4_t mfma<QL_BF16>(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <> QL_DEV f32x4_t mfma<QL_F16>(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Issue this wave's share of one operand tile (256 rows x 64 k starting at (row0, k0)) as
// 8 direct-to-LDS loads. Instruction j of wave w fills tile rows r0 = (4j + w) * 8 .. +7;
// lane l writes LDS bytes [16 l, 16 l + 16) of that 1 KiB span, i.e. row r0 + l/8,
// physical chunk l%8, which holds logical chunk (l%8) ^ (l/8) of the row.
// Addresses are a wave-uniform 64-bit base (SGPRs) plus a 32-bit lane offset; rows past the
// last one re-read the last row, never past it.
struct TileLoader {
  int wave;          // wave index, wave-uniform
  int rsub;          // lane / 8
  uint32_t chunk16;  // 16 * chunk, bytes
};

QL_DEV TileLoader make_loader() {
  TileLoader t;
  const int lane = threadIdx.x & 63;
  t.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  t.rsub = lane >> 3;
  t.chunk16 = (uint32_t)(((lane & 7) ^ t.rsub) * 16);
  return t;
}

template <int R8 = 8>  // tile rows / 32: 8 (256 rows) or 7 (224 rows)
QL_DEV void load_tile(const TileLoader& t, const uint16_t* __restrict__ X, int64_t ld,
                      int64_t row0, int64_t rows, int64_t k0, char* __restrict__ lds_tile) {
#pragma unroll
  for (int j = 0; j < R8; ++j) {
    const int r0 = (4 * j + t.wave) * 8;
    const int64_t grow0 = row0 + r0;
    const int64_t base_row = grow0 < rows ? grow0 : rows - 1;
    const int64_t r = (grow0 + t.rsub) < rows ? grow0 + t.rsub : rows - 1;
    const uint32_t off = (uint32_t)(r - base_row) * (uint32_t)(ld * 2) + t.chunk16;
    const char* base = reinterpret_cast<const char*>(X + base_row * ld + k0);
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)(base + off), (lds_ptr_t)(lds_tile + r0 * kRowBytes),
                                     16, 0, 0);
  }
}

// Tile coordinates of this workgroup: XCD-contiguous renumbering, then grouped raster.
QL_DEV void tile_of(int64_t tiles_m, int64_t tiles_n, int64_t& tm, int64_t& tn) {
  const int64_t total = tiles_m * tiles_n;
  const int64_t t = blockIdx.x;
  const int64_t q = total / 8, r = total % 8;
  const int64_t xcd = t % 8, idx = t / 8;
  const int64_t tt = xcd * q + (xcd < r ? xcd : r) + idx;
  const int64_t per_group = kGroupM * tiles_n;
  const int64_t g = tt / per_group;
  const int64_t first_m = g * kGroupM;
  const int64_t gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int64_t in_group = tt - g * per_group;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

// Fragment reads of one 32-k half of a stage: a[i] rows wm*128 + 16 i + fr, b[j] rows
// wn*16*NJ + 16 j + fr.
template <int NJ>
QL_DEV void read_frags(const char* __restrict__ stage, int half, int wm, int wn, int fr, int fq,
                       uint4 (&a)[8], uint4 (&b)[NJ]) {
  const char* as = stage + (wm * 128 + fr) * kRowBytes;
  const char* bs = stage + kTileBytes + (wn * 16 * NJ + fr) * kRowBytes;
  const int c = ((half * 4 + fq) ^ (fr & 7)) * 16;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = *reinterpret_cast<const uint4*>(as + i * 16 * kRowBytes + c);
    if (i < NJ) b[i] = *reinterpret_cast<const uint4*>(bs + i * 16 * kRowBytes + c);
  }
}

template <int IT, int NJ>
QL_DEV void mma_half(f32x4_t (&acc)[8][NJ], const uint4 (&a)[8], const uint4 (&b)[NJ]) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      acc[i][j] = mfma<IT>(b[j], a[i], acc[i][j]);
    }
}

// One K step kt, software-pipelined across steps. On entry f0 holds the first-half
// fragments of stage `cur` (read during the previous step) and the DMA of step kt+1 into
// `nxt` is in flight. The step reads the second half of `cur` while multiplying the first;
// then every wave waits for its DMA of step kt+1 and meets at the barrier (after it, all of
// `cur` has been read by every wave), issues the DMA of step kt+2 into `cur` (the last step
// reloads itself: in bounds, never read), and reads the first half of `nxt` while
// multiplying the second half of `cur`. `cur` and `nxt` are restrict-qualified so the
// compiler's wait-count pass does not make these reads wait for the DMA into `cur`.
// Per half step: R = 8 + NJ fragment reads, 8 NJ MFMAs, and (second half) R DMA loads.
template <int IT, int NJ>
QL_DEV void mma_step_pipe(f32x4_t (&acc)[8][NJ], uint4 (&f0a)[8], uint4 (&f0b)[NJ],
                          char* __restrict__ cur, char* __restrict__ nxt, const TileLoader& la,
                          const uint16_t* __restrict__ A2, int64_t lda2,
                          const uint16_t* __restrict__ B2, int64_t ldb2, int64_t k2, int64_t m0,
                          int64_t n0, int64_t M, int64_t N, int wm, int wn, int fr, int fq) {
  constexpr int R = 8 + NJ, MF = 8 * NJ;
  uint4 f1a[8], f1b[NJ];
  read_frags<NJ>(cur, 1, wm, wn, fr, fq, f1a, f1b);
  mma_half<IT, NJ>(acc, f0a, f0b);
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
  for (int t = 0; t < R; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, MF - 1 - 3 * R, 0);
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  load_tile(la, A2, lda2, m0, M, k2, cur);
  load_tile<NJ>(la, B2, ldb2, n0, N, k2, cur + kTileBytes);
  read_frags<NJ>(nxt, 0, wm, wn, fr, fq, f0a, f0b);
  mma_half<IT, NJ>(acc, f1a, f1b);
  __builtin_amdgcn_sched_group_barrier(0x020, R, 1);
#pragma unroll
  for (int t = 0; t < R; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 1);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, MF - 2 * R, 1);
}

// PARTIAL: write the raw fp32 sums of this split to ws[split][M][N]; otherwise the final
// alpha / beta / bias epilogue into C (type OT).
template <int IT, int OT, bool PARTIAL, int NJ>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_nt_kernel(const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ B,
                    int64_t ldb, const uint16_t* __restrict__ A2, int64_t lda2,
                    const uint16_t* __restrict__ B2, int64_t ldb2, int64_t K2,
                    typename Elem<OT>::T* __restrict__ C, int64_t ldc,
                    float* __restrict__ ws, const uint16_t* __restrict__ bias, int64_t M,
                    int64_t N, int64_t K, int64_t k_per_split, float alpha, float beta,
                    bool vec_out) {
  __shared__ __attribute__((aligned(1024))) char smem[2 * kStageBytes];
  constexpr int BN = bn_of<NJ>();
  int64_t tm, tn;
  tile_of((M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int64_t kb = (int64_t)blockIdx.y * k_per_split;
  const int64_t ke = (kb + k_per_split < K) ? kb + k_per_split : K;
  const int nk1 = (int)((ke - kb) / BK);
  // the second segment (A2 B2^T, K2 columns) is appended to the last split
  const int nk = nk1 + ((int)blockIdx.y == (int)gridDim.y - 1 ? (int)(K2 / BK) : 0);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 15;  // fragment row within a 16-row sub-tile
  const int fq = lane >> 4;  // fragment k quarter (8 k each) within a 32-k step

  f32x4_t acc[8][NJ];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const TileLoader la = make_loader();
  // k index of step t in its segment, and the segment's operands
  auto seg_k = [&](int t) -> int64_t { return t < nk1 ? kb + (int64_t)t * BK : (int64_t)(t - nk1) * BK; };
  if (nk > 0) {
    const bool s1 = nk1 > 0;
    load_tile(la, s1 ? A : A2, s1 ? lda : lda2, m0, M, seg_k(0), smem);
    load_tile<NJ>(la, s1 ? B : B2, s1 ? ldb : ldb2, n0, N, seg_k(0), smem + kTileBytes);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const int t1 = nk > 1 ? 1 : 0;
    const bool s1b = t1 < nk1;
    load_tile(la, s1b ? A : A2, s1b ? lda : lda2, m0, M, seg_k(t1), smem + kStageBytes);
    load_tile<NJ>(la, s1b ? B : B2, s1b ? ldb : ldb2, n0, N, seg_k(t1),
                  smem + kStageBytes + kTileBytes);
    uint4 f0a[8], f0b[NJ];
    read_frags<NJ>(smem, 0, wm, wn, fr, fq, f0a, f0b);
    for (int kt = 0; kt < nk; ++kt) {
      char* cur = smem + (kt & 1) * kStageBytes;
      char* nxt = smem + ((kt + 1) & 1) * kStageBytes;
      const int t2 = kt + 2 < nk ? kt + 2 : nk - 1;
      const bool s2 = t2 < nk1;
      mma_step_pipe<IT, NJ>(acc, f0a, f0b, cur, nxt, la, s2 ? A : A2, s2 ? lda : lda2, s2 ? B : B2,
                        s2 ? ldb : ldb2, seg_k(t2), m0, n0, M, N, wm, wn, fr, fq);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue: lane owns row fr of each 16-row sub-tile i and columns 4*fq .. 4*fq+3 of each
  // 16-column sub-tile j.
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t row = m0 + wm * 128 + i * 16 + fr;
    if (row >= M) continue;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t col = n0 + wn * 16 * NJ + j * 16 + 4 * fq;
      if (col >= N) continue;
      if constexpr (PARTIAL) {
        float* p = ws + ((int64_t)blockIdx.y * M + row) * N + col;
        if (col + 3 < N && (N & 3) == 0) {
          *reinterpret_cast<float4*>(p) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2],
                                                      acc[i][j][3]);
        } else {
          for (int e = 0; e < 4; ++e)
            if (col + e < N) p[e] = acc[i][j][e];
        }
      } else {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = alpha * acc[i][j][e];
        auto* cp = C + row * ldc + col;
        if (beta != 0.f)
          for (int e = 0; e < 4; ++e)
            if (col + e < N) v[e] += beta * Elem<OT>::to_f32(cp[e]);
        if (bias)
          for (int e = 0; e < 4; ++e)
            if (col + e < N) v[e] += Elem<IT>::to_f32(bias[col + e]);
        const bool vec = vec_out && col + 3 < N;
        if (vec) {
          if constexpr (OT == QL_F32) {
            *reinterpret_cast<float4*>(cp) = make_float4(v[0], v[1], v[2], v[3]);
          } else if constexpr (OT == QL_BF16) {
            *reinterpret_cast<uint2*>(cp) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
          } else {
            *reinterpret_cast<uint2*>(cp) = make_uint2(pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3]));
          }
        } else {
          for (int e = 0; e < 4; ++e)
            if (col + e < N) cp[e] = Elem<OT>::from_f32(v[e]);
        }
      }
    }
  }
}

// out[m, n] = alpha * sum_s ws[s][m][n] (+ beta * out) (+ bias[n]), summed in split order.
template <int IT, int OT>
__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ ws, int splits,
                                                     typename Elem<OT>::T* __restrict__ C,
                                                     int64_t ldc, const uint16_t* __restrict__ bias,
                                                     int64_t M, int64_t N, float alpha, float beta) {
  const int64_t total = M * N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    float s = 0.f;
    for (int z = 0; z < splits; ++z) s += ws[z * total + i];
    const int64_t row = i / N, col = i - row * N;
    float v = alpha * s;
    auto* cp = C + row * ldc + col;
    if (beta != 0.f) v += beta * Elem<OT>::to_f32(*cp);
    if (bias) v += Elem<IT>::to_f32(bias[col]);
    *cp = Elem<OT>::from_f32(v);
  }
}

template <int IT, int OT, int NJ>
int launch(const void* A, int64_t lda, const void* B, int64_t ldb, const void* A2, int64_t lda2,
           const void* B2, int64_t ldb2, int64_t K2, void* C, int64_t ldc, const void* bias,
           int64_t M, int64_t N, int64_t K, float alpha, float beta, int splits, float* ws,
           hipStream_t s) {
  using T = typename Elem<OT>::T;
  constexpr int BN = bn_of<NJ>();
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const int64_t kps = ((K / BK + splits - 1) / splits) * BK;
  const int nsplit = (int)((K + kps - 1) / kps);
  if (nsplit <= 1) {
    const bool vec_out = ql_aligned(C, 4 * ql_elem_size(OT)) && ldc % 4 == 0;
    hipLaunchKernelGGL((gemm_nt_kernel<IT, OT, false, NJ>), dim3((unsigned)tiles, 1), dim3(kThreads), 0, s,
                       (const uint16_t*)A, lda, (const uint16_t*)B, ldb, (const uint16_t*)A2,
                       lda2, (const uint16_t*)B2, ldb2, K2, (T*)C, ldc, nullptr,
                       (const uint16_t*)bias, M, N, K, K, alpha, beta, vec_out);
    return ql_launch_status();
  }
  hipLaunchKernelGGL((gemm_nt_kernel<IT, QL_F32, true, NJ>), dim3((unsigned)tiles, (unsigned)nsplit),
                     dim3(kThreads), 0, s,
                     (const uint16_t*)A, lda, (const uint16_t*)B, ldb, (const uint16_t*)A2, lda2,
                     (const uint16_t*)B2, ldb2, K2, (float*)nullptr, (int64_t)0,
                     ws, (const uint16_t*)nullptr, M, N, K, kps, 1.0f, 0.0f, false);
  int st = ql_launch_status();
  if (st != QL_OK) return st;
  const int64_t total = M * N;
  int64_t grid = (total + 255) / 256;
  if (grid > 256 * 16) grid = 256 * 16;
  hipLaunchKernelGGL((splitk_reduce<IT, OT>), dim3((unsigned)grid), dim3(256), 0, s, ws, nsplit,
                     (T*)C, ldc, (const uint16_t*)bias, M, N, alpha, beta);
  return ql_launch_status();
}

// Tile width for an M x N output: 224 (NJ = 7) when N is a multiple of 224, the output is
// large enough to run without split-K (>= 128 tiles of 256 x 256) and the narrower tiles take
// fewer (waves x tile width) on 256 CUs, else 256. The 4096 x 3584 outputs of the 7B step are
// 224 tiles of 256 x 256 (one partial wave) but exactly 256 tiles of 256 x 224. Small outputs
// are split over K instead, where narrower tiles only add operand traffic.
int choose_nj(int64_t M, int64_t N) {
  if (N % 224) return 8;
  const int64_t tm = (M + BM - 1) / BM;
  const int64_t t8 = tm * ((N + 255) / 256);
  if (t8 < 128) return 8;
  const int64_t w8 = (t8 + 255) / 256;
  const int64_t w7 = (tm * (N / 224) + 255) / 256;
  return w7 * 7 < w8 * 8 ? 7 : 8;
}

}  // namespace

bool ql_gemm_nt_fits(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* B,
                     int64_t ldb) {
  return M > 0 && N > 0 && K > 0 && K % BK == 0 && lda % 8 == 0 && ldb % 8 == 0 &&
         ql_aligned(A, 16) && ql_aligned(B, 16) && (M + BM - 1) / BM * ((N + 223) / 224) < (1 << 30);
}

int64_t ql_gemm_nt_workspace_floats(int64_t M, int64_t N, int splits) {
  return splits > 1 ? (int64_t)splits * M * N : 0;
}

int ql_gemm_nt_auto_splits(int64_t M, int64_t N, int64_t K) {
  // Enough workgroups for 256 CUs: split K while there are fewer tiles than CUs and each
  // split keeps at least 8 K steps.
  const int64_t bn = 32 * choose_nj(M, N);
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + bn - 1) / bn);
  int s = 1;
  while (tiles * s < 192 && (K / BK) / (2 * s) >= 8 && s < 64) s *= 2;
  return s;
}

int ql_gemm_nt2(int in_dtype, int c_dtype, int64_t M, int64_t N, int64_t K, const void* A,
                int64_t lda, const void* B, int64_t ldb, const void* A2, int64_t lda2,
                const void* B2, int64_t ldb2, int64_t K2, void* C, int64_t ldc, const void* bias,
                float alpha, float beta, int splits, float* ws, hipStream_t s) {
  if (splits > 1 && !ws) return QL_EINVAL;
  if (K2 < 0 || K2 % BK) return QL_EINVAL;
  if (K2 == 0) A2 = B2 = nullptr;
  const bool narrow = choose_nj(M, N) == 7;
#define QL_GEMM_NT_LAUNCH(ITC, NJC)                                                            \
  QL_DISPATCH_DTYPE(c_dtype, OT,                                                               \
                    return (launch<ITC, OT, NJC>(A, lda, B, ldb, A2, lda2, B2, ldb2, K2, C, ldc, \
                                                 bias, M, N, K, alpha, beta, splits, ws, s)))
  if (in_dtype == QL_BF16) {
    if (narrow) {
      QL_GEMM_NT_LAUNCH(QL_BF16, 7);
    } else {
      QL_GEMM_NT_LAUNCH(QL_BF16, 8);
    }
  } else if (in_dtype == QL_F16) {
    if (narrow) {
      QL_GEMM_NT_LAUNCH(QL_F16, 7);
    } else {
      QL_GEMM_NT_LAUNCH(QL_F16, 8);
    }
  }
#undef QL_GEMM_NT_LAUNCH
  return QL_EDTYPE;
}

int ql_gemm_nt(int in_dtype, int c_dtype, int64_t M, int64_t N, int64_t K, const void* A,
               int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, const void* bias,
               float alpha, float beta, int splits, float* ws, hipStream_t s) {
  return ql_gemm_nt2(in_dtype, c_dtype, M, N, K, A, lda, B, ldb, nullptr, 0, nullptr, 0, 0, C,
                     ldc, bias, alpha, beta, splits, ws, s);
}
