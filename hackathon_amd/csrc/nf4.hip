// NF4 dequantisation with a double-quantised absmax, for gfx950.
//
// Reference semantics: solution/nf4.py:25-49 (nf4_dequant_kernel) and :71-92
// (dequantize_nf4). Weight j lives in packed byte j/2 (high nibble first); its block scale
// is, with double quantisation,
//     s = code2[absmax_q[j / bs]] * absmax2[(j / bs) / bs2];   s = s + offset
// (two fp32 roundings, never an FMA), otherwise s = absmax[j / bs]. The weight is the fp32
// product nf4[nibble] * s, rounded once to the output dtype.
//
// HBM-bound: 0.5 B of nibbles + 1/bs B of absmax codes in, 2 B of bf16 out per weight.
// Fast path: one lane turns one 32-bit word (4 packed bytes = 8 weights) into one 16-byte
// bf16 store. Lanes of a wave take consecutive words, so each global load instruction reads
// 256 contiguous bytes and each store instruction writes 1 KiB contiguous; a workgroup
// covers UNROLL such spans with all loads issued before the first store. The 16-entry
// codebook and the 256-entry code2 table sit in LDS.
// The 16-bit outputs are written with nontemporal stores: the dequantised weight is 80% of
// the traffic and is not re-read by this kernel, and streaming it past the caches measured
// 1.7x faster on MI355X than ordinary stores (24.8 vs 44.4 us for 18944 x 3584). Each such
// store instruction covers whole 128-B lines (64 lanes x 16 B contiguous); nontemporal
// stores that leave partial lines were measured far slower, so fp32 output (two 16-B
// stores per lane, 32 B apart) keeps ordinary stores.
#include "ql_common.h"

namespace {

constexpr int kThreads = 256;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int OUT_DT> struct Group8;  // 8 dequantised weights -> one vector store
template <> struct Group8<QL_BF16> {
  static QL_DEV void store(uint16_t* out, int64_t g, const float* w) {
    const u32x4 v = {pack_bf16x2(w[0], w[1]), pack_bf16x2(w[2], w[3]), pack_bf16x2(w[4], w[5]),
                     pack_bf16x2(w[6], w[7])};
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(out) + g);
  }
};
template <> struct Group8<QL_F16> {
  static QL_DEV void store(uint16_t* out, int64_t g, const float* w) {
    const u32x4 v = {pack_f16x2(w[0], w[1]), pack_f16x2(w[2], w[3]), pack_f16x2(w[4], w[5]),
                     pack_f16x2(w[6], w[7])};
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(out) + g);
  }
};
template <> struct Group8<QL_F32> {
  static QL_DEV void store(float* out, int64_t g, const float* w) {
    float4* o = reinterpret_cast<float4*>(out) + 2 * g;
    o[0] = make_float4(w[0], w[1], w[2], w[3]);
    o[1] = make_float4(w[4], w[5], w[6], w[7]);
  }
};

// The fp32 product must be rounded to fp32 before the conversion to the output type. The
// AMDGPU backend otherwise fuses (fptrunc (fmul a b)) into one v_fma_mixlo_f16 with a single
// rounding (also under -ffp-contract=off); an empty register barrier keeps the two steps.
QL_DEV float fp32_rounded(float x) {
  asm("" : "+v"(x));
  return x;
}

// Block scale of block `blk`, exactly as the reference orders the fp32 operations.
template <bool NESTED>
QL_DEV float block_scale(int64_t blk, const uint8_t* __restrict__ absmax_q,
                         const float* __restrict__ absmax_f, const float* code2_lds,
                         const float* __restrict__ absmax2, float offset, int log2_bs2) {
#pragma clang fp contract(off)
  if constexpr (NESTED) {
    float s = code2_lds[absmax_q[blk]] * absmax2[blk >> log2_bs2];
    return s + offset;
  } else {
    return absmax_f[blk];
  }
}

// One workgroup's span of the vector path: groups tile * kThreads * UNROLL + [0, kThreads *
// UNROLL) of one weight.
template <int OUT_DT, bool NESTED, int UNROLL>
QL_DEV void dequant_vec_span(int64_t tile, const uint32_t* __restrict__ packed4, int64_t n_groups,
                             const uint8_t* __restrict__ absmax_q,
                             const float* __restrict__ absmax_f, const float* __restrict__ code2,
                             const float* __restrict__ absmax2, float offset, int log2_bs,
                             int log2_bs2, const float* __restrict__ nf4_table,
                             typename Elem<OUT_DT>::T* __restrict__ out) {
#pragma clang fp contract(off)
  __shared__ float table[16];
  __shared__ float code2_lds[NESTED ? 256 : 1];
  // Every global load this thread needs is issued before the table fill and its barrier,
  // so their latencies overlap (the kernel is latency-bound at small weights); the table
  // loads go first because loads complete in issue order.
  const float tab_v = threadIdx.x < 16 ? nf4_table[threadIdx.x] : 0.f;
  const float code2_v = NESTED ? code2[threadIdx.x] : 0.f;  // kThreads == 256
  const int64_t base = tile * (kThreads * UNROLL) + threadIdx.x;
  uint32_t word[UNROLL];
  uint32_t code[UNROLL];  // absmax code (nested) or the fp32 absmax bits (plain)
  float scale2[UNROLL];   // second-level scale (nested)
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t g = base + (int64_t)u * kThreads;
    const bool ok = g < n_groups;
    const int64_t blk = ok ? (g * 8) >> log2_bs : 0;  // a group's 8 weights share a block
    word[u] = ok ? packed4[g] : 0u;
    if constexpr (NESTED) {
      code[u] = absmax_q[blk];
      scale2[u] = absmax2[blk >> log2_bs2];
    } else {
      code[u] = __float_as_uint(absmax_f[blk]);
      scale2[u] = 0.f;
    }
  }
  if (threadIdx.x < 16) table[threadIdx.x] = tab_v;
  if constexpr (NESTED) code2_lds[threadIdx.x] = code2_v;
  __syncthreads();
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t g = base + (int64_t)u * kThreads;
    if (g >= n_groups) continue;
    float s;
    if constexpr (NESTED) {
      s = code2_lds[code[u]] * scale2[u];  // two fp32 roundings, as the reference orders them
      s = s + offset;
    } else {
      s = __uint_as_float(code[u]);
    }
    float w[8];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t byte = (word[u] >> (8 * b)) & 0xffu;
      w[2 * b] = fp32_rounded(table[byte >> 4] * s);      // high nibble: the first weight
      w[2 * b + 1] = fp32_rounded(table[byte & 15u] * s);  // low nibble: the second
    }
    Group8<OUT_DT>::store(out, g, w);
  }
}

template <int OUT_DT, bool NESTED, int UNROLL>
__global__ __launch_bounds__(kThreads) void nf4_dequant_vec(
    const uint32_t* __restrict__ packed4, int64_t n_groups, const uint8_t* __restrict__ absmax_q,
    const float* __restrict__ absmax_f, const float* __restrict__ code2,
    const float* __restrict__ absmax2, float offset, int log2_bs, int log2_bs2,
    const float* __restrict__ nf4_table, typename Elem<OUT_DT>::T* __restrict__ out) {
  dequant_vec_span<OUT_DT, NESTED, UNROLL>(blockIdx.x, packed4, n_groups, absmax_q, absmax_f,
                                           code2, absmax2, offset, log2_bs, log2_bs2, nf4_table,
                                           out);
}

// Several weights in one launch (the q/k/v or gate/up projections of a layer): one launch
// instead of one per weight, so the small weights' latency-bound ramps overlap with the large
// ones'. Weight i owns workgroups [tile_begin_i, tile_begin_{i+1}); the descriptor table
// travels by value in the kernel arguments and each workgroup selects its entry with
// wave-uniform compares.
constexpr int kMaxGroup = 4;
struct DqItem {
  const uint8_t* packed;
  const uint8_t* absmax_q;
  const float* absmax_f;
  const float* code2;
  const float* absmax2;
  void* out;
  int64_t rows;      // vector path: the weight's 4-byte groups; transposed path: rows
  int64_t cols;      // transposed path only
  float offset;
  int log2_bs, log2_bs2;
  uint32_t tile_begin;  // first workgroup (x index) of this weight
};
struct DqGroup {
  DqItem item[kMaxGroup];
  int count;
};

QL_DEV DqItem pick_item(const DqGroup& grp, uint32_t bx) {
  DqItem it = grp.item[0];
#pragma unroll
  for (int j = 1; j < kMaxGroup; ++j)
    if (j < grp.count && bx >= grp.item[j].tile_begin) it = grp.item[j];
  return it;
}

template <int OUT_DT, bool NESTED, int UNROLL>
__global__ __launch_bounds__(kThreads) void nf4_dequant_vec_group(
    const DqGroup grp, const float* __restrict__ nf4_table) {
  const DqItem it = pick_item(grp, blockIdx.x);
  dequant_vec_span<OUT_DT, NESTED, UNROLL>(
      blockIdx.x - it.tile_begin, reinterpret_cast<const uint32_t*>(it.packed), it.rows,
      it.absmax_q, it.absmax_f, it.code2, it.absmax2, it.offset, it.log2_bs, it.log2_bs2,
      nf4_table, static_cast<typename Elem<OUT_DT>::T*>(it.out));
}

// Any even blocksize, any alignment: one thread per packed byte.
template <int OUT_DT, bool NESTED>
__global__ __launch_bounds__(kThreads) void nf4_dequant_scalar(
    const uint8_t* __restrict__ packed, int64_t byte_begin, int64_t byte_end,
    const uint8_t* __restrict__ absmax_q, const float* __restrict__ absmax_f,
    const float* __restrict__ code2, const float* __restrict__ absmax2, float offset,
    int64_t blocksize, int64_t blocksize2, const float* __restrict__ nf4_table,
    typename Elem<OUT_DT>::T* __restrict__ out) {
#pragma clang fp contract(off)
  const int64_t i = byte_begin + (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= byte_end) return;
  const int64_t blk = (2 * i) / blocksize;
  float s;
  if constexpr (NESTED) {
    s = code2[absmax_q[blk]] * absmax2[blk / blocksize2];
    s = s + offset;
  } else {
    s = absmax_f[blk];
  }
  const uint32_t byte = packed[i];
  Elem<OUT_DT>::store(out, 2 * i, fp32_rounded(nf4_table[byte >> 4] * s));
  Elem<OUT_DT>::store(out, 2 * i + 1, fp32_rounded(nf4_table[byte & 15u] * s));
}

// Transposed dequantisation: outT[k][n] = W[n][k] for W [rows, cols] (row-major, packed two
// per byte along k). The backward of the 4-bit linear needs dY @ W; with W^T stored [cols,
// rows] that contraction is k-contiguous on both operands. One workgroup per tile of 64 rows
// (n) x 128 columns (k). The packed tile (64 rows x 64 B) comes in with one coalesced 16-B
// load per thread (4 lanes per row) into LDS rows of 17 words (an odd stride: the row reads
// below meet distinct banks). Thread t then dequantises 16 consecutive k of the rows 2p and
// 2p+1 (p = t % 32, k-chunk t / 32), packs each (n, n+1) pair into one 32-bit LDS word of
// the [k][n] tile, and the tile leaves as 128 rows of 64 n = 128 contiguous bytes each,
// written with nontemporal 16-B stores (8 lanes per row). Same per-weight arithmetic as
// above, so outT is bit-identical to the transpose of the plain dequantisation.
constexpr int kTRows = 64, kTCols = 128;
constexpr int kTStride = 36;  // LDS words per k-row of the tile (32 used, 16-B aligned rows)
constexpr int kTInStride = 17;  // LDS words per packed input row (16 used)

// One 64 x 128 tile (n-tile nt, k-tile kt) of the transposed dequantisation.
template <int OUT_DT, bool NESTED>
QL_DEV void dequant_t_tile(int64_t nt, int64_t kt, const uint8_t* __restrict__ packed,
                           int64_t rows, int64_t cols, const uint8_t* __restrict__ absmax_q,
                           const float* __restrict__ absmax_f, const float* __restrict__ code2,
                           const float* __restrict__ absmax2, float offset, int log2_bs,
                           int log2_bs2, const float* __restrict__ nf4_table,
                           uint16_t* __restrict__ outT, int64_t ld_out) {
#pragma clang fp contract(off)
  __shared__ float table[16];
  __shared__ float code2_lds[NESTED ? 256 : 1];
  __shared__ __attribute__((aligned(16))) uint32_t tile[kTCols * kTStride];
  __shared__ uint32_t tile_in[kTRows * kTInStride];
  // n-tiles vary fastest: workgroups running together write adjacent 128-B pieces of the same
  // output rows (whole DRAM pages) instead of one piece each of many rows
  const int64_t n0 = nt * kTRows;
  const int64_t k0 = kt * kTCols;
  {  // packed input: thread t loads 16 B of row t / 4 (chunk t % 4)
    const int r = threadIdx.x >> 2, c = threadIdx.x & 3;
    if (n0 + r < rows) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(packed + ((n0 + r) * cols + k0) / 2 + 16 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) tile_in[r * kTInStride + 4 * c + e] = v[e];
    }
  }
  if (threadIdx.x < 16) table[threadIdx.x] = nf4_table[threadIdx.x];
  if constexpr (NESTED) code2_lds[threadIdx.x] = code2[threadIdx.x];  // kThreads == 256
  __syncthreads();

  const int p = threadIdx.x & 31, kc = threadIdx.x >> 5;
  const int64_t k = k0 + 16 * kc;
  float w[2][16];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t n = n0 + 2 * p + h;
    if (n < rows) {
      const int64_t j = n * cols + k;  // first weight index; j % 16 == 0
      const uint32_t* src = tile_in + (2 * p + h) * kTInStride + 2 * kc;
      const uint2 b = make_uint2(src[0], src[1]);
      const float s =
          block_scale<NESTED>(j >> log2_bs, absmax_q, absmax_f, code2_lds, absmax2, offset, log2_bs2);
      const uint32_t bw[2] = {b.x, b.y};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint32_t byte = (bw[q >> 2] >> (8 * (q & 3))) & 0xffu;
        w[h][2 * q] = fp32_rounded(table[byte >> 4] * s);
        w[h][2 * q + 1] = fp32_rounded(table[byte & 15u] * s);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) w[h][q] = 0.f;
    }
  }
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const uint32_t v = OUT_DT == QL_BF16 ? pack_bf16x2(w[0][q], w[1][q]) : pack_f16x2(w[0][q], w[1][q]);
    tile[(16 * kc + q) * kTStride + p] = v;
  }
  __syncthreads();
  const int c = threadIdx.x & 7;
  const int64_t n = n0 + 8 * c;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int kr = (threadIdx.x >> 3) + 32 * i;
    if (n < rows) {  // rows % 8 == 0: a 16-B chunk is entirely in or out
      const u32x4 v = *reinterpret_cast<const u32x4*>(&tile[kr * kTStride + 4 * c]);
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(outT + (k0 + kr) * ld_out + n));
    }
  }
}

template <int OUT_DT, bool NESTED>
__global__ __launch_bounds__(kThreads) void nf4_dequant_t_kernel(
    const uint8_t* __restrict__ packed, int64_t rows, int64_t cols,
    const uint8_t* __restrict__ absmax_q, const float* __restrict__ absmax_f,
    const float* __restrict__ code2, const float* __restrict__ absmax2, float offset, int log2_bs,
    int log2_bs2, const float* __restrict__ nf4_table, uint16_t* __restrict__ outT,
    int64_t ld_out) {
  dequant_t_tile<OUT_DT, NESTED>(blockIdx.x, blockIdx.y, packed, rows, cols, absmax_q, absmax_f,
                                 code2, absmax2, offset, log2_bs, log2_bs2, nf4_table, outT,
                                 ld_out);
}

// Grouped transposed dequantisation: weight i's n-tiles are x indices [tile_begin_i, ..) and
// its output block starts at item.out (its column offset in the shared out_t); the k-tiles
// (y) run to the widest weight and a narrower weight's surplus workgroups exit at once.
template <int OUT_DT, bool NESTED>
__global__ __launch_bounds__(kThreads) void nf4_dequant_t_group(
    const DqGroup grp, const float* __restrict__ nf4_table, int64_t ld_out) {
  const DqItem it = pick_item(grp, blockIdx.x);
  if ((int64_t)blockIdx.y * kTCols >= it.cols) return;  // whole workgroup, before any barrier
  dequant_t_tile<OUT_DT, NESTED>(blockIdx.x - it.tile_begin, blockIdx.y, it.packed, it.rows,
                                 it.cols, it.absmax_q, it.absmax_f, it.code2, it.absmax2,
                                 it.offset, it.log2_bs, it.log2_bs2, nf4_table,
                                 static_cast<uint16_t*>(it.out), ld_out);
}

int ilog2_exact(int64_t v) {  // log2 of a power of two, else -1
  if (v <= 0 || (v & (v - 1))) return -1;
  int l = 0;
  while ((int64_t(1) << l) < v) ++l;
  return l;
}

template <int OUT_DT, bool NESTED>
int launch_dequant(const uint8_t* packed, int64_t n_weights, const void* absmax,
                   const float* code2, const float* absmax2, float offset, int blocksize,
                   int blocksize2, const float* table, void* out_v, hipStream_t stream) {
  using T = typename Elem<OUT_DT>::T;
  T* out = static_cast<T*>(out_v);
  const uint8_t* aq = NESTED ? static_cast<const uint8_t*>(absmax) : nullptr;
  const float* af = NESTED ? nullptr : static_cast<const float*>(absmax);
  const int64_t n_bytes = n_weights / 2;
  const int lbs = ilog2_exact(blocksize);
  const int lbs2 = NESTED ? ilog2_exact(blocksize2) : 0;
  const bool fast = lbs >= 3 && lbs2 >= 0 && ql_aligned(packed, 4) && ql_aligned(out, 16);
  int64_t done = 0;
  if (fast) {
    const int64_t n_groups = n_bytes / 4;
    // Two words per lane at every size: measured best on MI355X from the 0.5B weight
    // (4864 x 896, 3.4 us per launch, where one word per lane took 3.8 us) to the 7B gate
    // weight (18944 x 3584, 25 us).
    if (n_groups > 0) {
      const int64_t grid = (n_groups + kThreads * 2 - 1) / (kThreads * 2);
      hipLaunchKernelGGL((nf4_dequant_vec<OUT_DT, NESTED, 2>), dim3((unsigned)grid),
                         dim3(kThreads), 0, stream, reinterpret_cast<const uint32_t*>(packed),
                         n_groups, aq, af, code2, absmax2, offset, lbs, lbs2, table, out);
    }
    done = n_groups * 4;
  }
  if (done < n_bytes) {
    const int64_t grid = (n_bytes - done + kThreads - 1) / kThreads;
    hipLaunchKernelGGL((nf4_dequant_scalar<OUT_DT, NESTED>), dim3((unsigned)grid), dim3(kThreads),
                       0, stream, packed, done, n_bytes, aq, af, code2, absmax2, offset,
                       (int64_t)blocksize, (int64_t)(NESTED ? blocksize2 : 1), table, out);
  }
  return ql_launch_status();
}

}  // namespace

extern "C" int qlora_nf4_dequant(const uint8_t* packed, int64_t n_weights, const void* absmax,
                                 int nested, const float* code2, const float* absmax2,
                                 float offset, int blocksize, int blocksize2,
                                 const float* nf4_table, void* out, int out_dtype,
                                 ql_stream_t stream) {
  if (n_weights < 0 || (n_weights & 1) || blocksize < 2 || (blocksize & 1)) return QL_EINVAL;
  if (n_weights == 0) return QL_OK;
  if (!packed || !absmax || !nf4_table || !out) return QL_EINVAL;
  if (nested && (!code2 || !absmax2 || blocksize2 < 2 || (blocksize2 & 1))) return QL_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (nested) {
    QL_DISPATCH_DTYPE(out_dtype, DT,
                      return launch_dequant<DT, true>(packed, n_weights, absmax, code2, absmax2,
                                                      offset, blocksize, blocksize2, nf4_table,
                                                      out, s));
  } else {
    QL_DISPATCH_DTYPE(out_dtype, DT,
                      return launch_dequant<DT, false>(packed, n_weights, absmax, nullptr,
                                                       nullptr, 0.f, blocksize, 1, nf4_table, out,
                                                       s));
  }
  return QL_EDTYPE;
}

extern "C" int qlora_nf4_dequant_t(const uint8_t* packed, int64_t rows, int64_t cols,
                                   const void* absmax, int nested, const float* code2,
                                   const float* absmax2, float offset, int blocksize,
                                   int blocksize2, const float* nf4_table, void* out_t,
                                   int64_t ld_out, int out_dtype, ql_stream_t stream) {
  if (rows < 0 || cols < 0 || ld_out < rows) return QL_EINVAL;
  if (rows == 0 || cols == 0) return QL_OK;
  if (!packed || !absmax || !nf4_table || !out_t) return QL_EINVAL;
  if (out_dtype != QL_BF16 && out_dtype != QL_F16) return QL_EDTYPE;
  const int lbs = ilog2_exact(blocksize);
  if (lbs < 4) return QL_EINVAL;  // a power of two >= 16
  if (nested && (!code2 || !absmax2 || ilog2_exact(blocksize2) < 0)) return QL_EINVAL;
  if (cols % kTCols || rows % 8 || ld_out % 8) return QL_ESHAPE;
  if (!ql_aligned(packed, 16) || !ql_aligned(out_t, 16)) return QL_EALIGN;
  const int lbs2 = nested ? ilog2_exact(blocksize2) : 0;
  if ((rows + kTRows - 1) / kTRows > INT32_MAX || cols / kTCols > 65535) return QL_ESHAPE;
  const dim3 grid((unsigned)((rows + kTRows - 1) / kTRows), (unsigned)(cols / kTCols));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* aq = nested ? static_cast<const uint8_t*>(absmax) : nullptr;
  const float* af = nested ? nullptr : static_cast<const float*>(absmax);
  uint16_t* o = static_cast<uint16_t*>(out_t);
#define QL_DQT(DT, NST)                                                                        \
  hipLaunchKernelGGL((nf4_dequant_t_kernel<DT, NST>), grid, dim3(kThreads), 0, s, packed, rows, \
                     cols, aq, af, code2, absmax2, offset, lbs, lbs2, nf4_table, o, ld_out)
  if (out_dtype == QL_BF16) {
    if (nested) QL_DQT(QL_BF16, true); else QL_DQT(QL_BF16, false);
  } else {
    if (nested) QL_DQT(QL_F16, true); else QL_DQT(QL_F16, false);
  }
#undef QL_DQT
  return ql_launch_status();
}

namespace {

// Checks one weight of a group as the single-weight entries check theirs and fills its scale
// fields; `transposed` applies qlora_nf4_dequant_t's extra shape rules.
int group_item(const ql_nf4_weight& w, int nested, bool transposed, int64_t ld_out,
               DqItem* it) {
  if (w.rows < 0 || w.cols < 0) return QL_EINVAL;
  if (w.rows == 0 || w.cols == 0) return QL_OK;
  if (!w.packed || !w.absmax || !w.out) return QL_EINVAL;
  if (nested && (!w.code2 || !w.absmax2)) return QL_EINVAL;
  it->packed = w.packed;
  it->absmax_q = nested ? static_cast<const uint8_t*>(w.absmax) : nullptr;
  it->absmax_f = nested ? nullptr : static_cast<const float*>(w.absmax);
  it->code2 = nested ? w.code2 : nullptr;
  it->absmax2 = nested ? w.absmax2 : nullptr;
  it->offset = nested ? w.offset : 0.f;
  it->out = w.out;
  it->cols = w.cols;
  it->log2_bs = ilog2_exact(w.blocksize);
  it->log2_bs2 = nested ? ilog2_exact(w.blocksize2) : 0;
  if (transposed) {
    if (it->log2_bs < 4 || it->log2_bs2 < 0) return QL_EINVAL;
    if (ld_out < w.rows) return QL_EINVAL;
    if (w.cols % kTCols || w.rows % 8) return QL_ESHAPE;
    if (!ql_aligned(w.packed, 16) || !ql_aligned(w.out, 16)) return QL_EALIGN;
    it->rows = w.rows;
  } else {
    if (w.cols > INT64_MAX / w.rows) return QL_EINVAL;
    const int64_t n = w.rows * w.cols;
    if (it->log2_bs < 3 || it->log2_bs2 < 0) return QL_EINVAL;  // powers of two, blocksize >= 8
    if (n % 8) return QL_ESHAPE;
    if (!ql_aligned(w.packed, 4) || !ql_aligned(w.out, 16)) return QL_EALIGN;
    it->rows = n / 8;  // 4-byte groups
  }
  return QL_OK;
}

template <int OUT_DT, bool NESTED>
void launch_group(const DqGroup& grp, uint32_t tiles, const float* table, hipStream_t s) {
  hipLaunchKernelGGL((nf4_dequant_vec_group<OUT_DT, NESTED, 2>), dim3(tiles), dim3(kThreads), 0,
                     s, grp, table);
}

}  // namespace

extern "C" int qlora_nf4_dequant_group(const ql_nf4_weight* weights, int count, int nested,
                                       const float* nf4_table, int out_dtype,
                                       ql_stream_t stream) {
  if (count < 1 || count > kMaxGroup || !weights || !nf4_table) return QL_EINVAL;
  DqGroup grp{};
  int64_t tiles = 0;
  for (int i = 0; i < count; ++i) {
    DqItem it{};
    const int st = group_item(weights[i], nested, false, 0, &it);
    if (st != QL_OK) return st;
    if (it.rows == 0 || weights[i].rows == 0 || weights[i].cols == 0) continue;
    it.tile_begin = (uint32_t)tiles;
    tiles += (it.rows + kThreads * 2 - 1) / (kThreads * 2);
    if (tiles > INT32_MAX) return QL_ESHAPE;
    grp.item[grp.count++] = it;
  }
  if (grp.count == 0) return QL_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (nested) {
    QL_DISPATCH_DTYPE(out_dtype, DT, launch_group<DT, true>(grp, (uint32_t)tiles, nf4_table, s));
  } else {
    QL_DISPATCH_DTYPE(out_dtype, DT, launch_group<DT, false>(grp, (uint32_t)tiles, nf4_table, s));
  }
  return ql_launch_status();
}

extern "C" int qlora_nf4_dequant_t_group(const ql_nf4_weight* weights, int count, int nested,
                                         const float* nf4_table, int64_t ld_out, int out_dtype,
                                         ql_stream_t stream) {
  if (count < 1 || count > kMaxGroup || !weights || !nf4_table) return QL_EINVAL;
  if (out_dtype != QL_BF16 && out_dtype != QL_F16) return QL_EDTYPE;
  if (ld_out % 8) return QL_ESHAPE;
  DqGroup grp{};
  int64_t tiles = 0, max_cols = 0;
  for (int i = 0; i < count; ++i) {
    DqItem it{};
    const int st = group_item(weights[i], nested, true, ld_out, &it);
    if (st != QL_OK) return st;
    if (weights[i].rows == 0 || weights[i].cols == 0) continue;
    it.tile_begin = (uint32_t)tiles;
    tiles += (it.rows + kTRows - 1) / kTRows;
    if (tiles > INT32_MAX) return QL_ESHAPE;
    max_cols = it.cols > max_cols ? it.cols : max_cols;
    grp.item[grp.count++] = it;
  }
  if (grp.count == 0) return QL_OK;
  if (max_cols / kTCols > 65535) return QL_ESHAPE;
  const dim3 grid((unsigned)tiles, (unsigned)(max_cols / kTCols));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define QL_DQTG(DT, NST)                                                                      \
  hipLaunchKernelGGL((nf4_dequant_t_group<DT, NST>), grid, dim3(kThreads), 0, s, grp, nf4_table, \
                     ld_out)
  if (out_dtype == QL_BF16) {
    if (nested) QL_DQTG(QL_BF16, true); else QL_DQTG(QL_BF16, false);
  } else {
    if (nested) QL_DQTG(QL_F16, true); else QL_DQTG(QL_F16, false);
  }
#undef QL_DQTG
  return ql_launch_status();
}
