// Causal flash attention, forward and backward, for the QLoRA step on CDNA4 matrix cores.
//
// The reference step runs attention through torch's scaled_dot_product_attention
// (transformers/models/qwen2/modeling_qwen2.py:220, the SDPA path of Qwen2Attention); these
// kernels are the native replacement: O = softmax(Q K^T * scale, causal) V with grouped-query
// heads, 16-bit in and out, fp32 accumulation and softmax, and the row log-sum-exp kept for
// the backward. The backward follows the FlashAttention-2 split: dQ per query block, which also
// forms Delta = rowsum(dO * O) for its rows, then dK, dV per key block, each recomputing P from
// Q, K and the lse.
//
// Building blocks shared by every kernel:
//  - v_mfma_f32_16x16x32 (bf16 or fp16). A pair of C tiles stacked along their rows is itself
//    an MFMA operand whose contraction index is that row index (the order inside a 32-step is
//    a permutation, applied identically to the other operand), so P, P^T, dS and dS^T feed
//    the next product straight from registers.
//  - 64-row x 128-d tiles (256-B rows) moved global -> LDS by direct-to-LDS loads (no VGPR
//    staging), with the 16-B chunks of row r XOR-swizzled by f(r) = 4 ((r >> 1) & 3) | 3 (r & 1)
//    (values 0 3 4 7 8 11 12 15 on any 8 aligned rows). One LDS copy of a matrix serves the
//    matrix and its transpose without bank conflicts, as measured with SQ_LDS_BANK_CONFLICT on
//    gfx950 (64 banks, 256 B a cycle):
//      ds_read_b128 row fragments (lane l reads row l % 16, logical chunk c + l / 16): the
//      lanes served together are not lanes 0..15 (a swizzle bijective on 16 rows still costs
//      4 stall cycles per read); every probe fits 8-lane blocks b and b ^ 3 sharing a cycle
//      (lanes 0..7 with 24..31, 8..15 with 16..23), so f(r) and f(r) ^ 1 must not meet over
//      8 aligned rows: bits 1..3 of f run through all 8 values;
//      ds_read_b64_tr_b16 (32 lanes a cycle on 8 consecutive rows x 32 B): f >> 1 distinct
//      over 8 aligned rows, the same condition.
//    Swizzles meeting only one condition left the dK/dV kernel at 1.2 to 2.45 bank-conflict
//    stall cycles per LDS instruction.
//  - two LDS stages per kernel: the next block's DMA runs under the current block's math,
//    with one barrier per block.
//  - 4 waves per workgroup and at most 256 registers per lane, so two workgroups share a CU.
// Head dim 128; any sequence length (rows and keys past the end are masked and clamped).
#include "ql_vec.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) void* gbl_ptr_t;
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

constexpr int HD = 128;                         // head dim
constexpr int kRows = 64;                       // rows per LDS tile / key block
constexpr int kRowBytes = HD * 2;               // 256
constexpr int kTileBytes = kRows * kRowBytes;   // 16 KiB
constexpr int BQ = 128;                         // forward, dQ: query rows per workgroup
constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Lazy rescaling threshold (log2 units): the running max m is only raised when a block's max
// exceeds it by more than this, so P = exp2(x - m) <= 2^8 stays well inside fp32 and bf16.
constexpr float kTau = 8.0f;

template <int DT> QL_DEV f32x4_t mfma(const uint4& a, const uint4& b, f32x4_t c);
template <> QL_DEV f32x4_t mfma<QL_BF16>(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <> QL_DEV f32x4_t mfma<QL_F16>(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

template <int DT> QL_DEV uint32_t pack2(float lo, float hi) {
  if constexpr (DT == QL_BF16) return pack_bf16x2(lo, hi);
  else return pack_f16x2(lo, hi);
}

// Two stacked C tiles (rows 0-15 and 16-31 of a 32-step) as one 16-bit operand.
template <int DT> QL_DEV uint4 pack_pair(const f32x4_t& a, const f32x4_t& c) {
  return make_uint4(pack2<DT>(a[0], a[1]), pack2<DT>(a[2], a[3]), pack2<DT>(c[0], c[1]),
                    pack2<DT>(c[2], c[3]));
}

QL_DEV f32x4_t zero4() { return f32x4_t{0.f, 0.f, 0.f, 0.f}; }

// ---- The direct-to-LDS ordering rule, and its check ------------------------------------------
// Every kernel here keeps one rule for the tiles its direct-to-LDS loads (dma_b128) fill: a
// tile is read only after the next wait_all_barrier (the loads are hidden from the compiler,
// so nothing else waits for them), and no load writes a tile that any wave may still read
// before that barrier. Built with -DQL_DMA_CHECK (the GPU tests build such a library beside
// the release one), each workgroup records in LDS which 1-KiB spans were loaded and which were
// read since the last wait_all_barrier; at every wait_all_barrier a span in both sets counts
// as a violation in a device counter (qlora_debug_dma_violations). Release builds compile the
// hooks to nothing.
#ifdef QL_DMA_CHECK
constexpr int kSpanWords = 160 / 32;  // 160 KiB of LDS in 1-KiB spans
__shared__ uint32_t dma_loaded[kSpanWords], dma_read[kSpanWords];
__device__ unsigned long long g_dma_violations;
QL_DEV void dma_mark(uint32_t* set, const void* p) {
  const uint32_t span = (uint32_t)(uintptr_t)(lds_ptr_t)p >> 10;
  atomicOr(&set[span >> 5], 1u << (span & 31));
}
QL_DEV void dma_ledger_clear() {
  if (threadIdx.x < kSpanWords) dma_loaded[threadIdx.x] = dma_read[threadIdx.x] = 0;
}
// every wave has passed the barrier: count the phase's overlaps, clear, meet again so that
// no wave marks the next phase before the clear
QL_DEV void dma_ledger_settle() {
  if (threadIdx.x < kSpanWords) {
    const uint32_t both = dma_loaded[threadIdx.x] & dma_read[threadIdx.x];
    if (both) atomicAdd(&g_dma_violations, (unsigned long long)__popc(both));
  }
  dma_ledger_clear();
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
#define QL_DMA_BEGIN() (dma_ledger_clear(), __syncthreads())
#define QL_DMA_LOADED(p) dma_mark(dma_loaded, (p))
#define QL_DMA_READ(p) dma_mark(dma_read, (p))
#define QL_DMA_SETTLE() dma_ledger_settle()
#else
#define QL_DMA_BEGIN() ((void)0)
#define QL_DMA_LOADED(p) ((void)0)
#define QL_DMA_READ(p) ((void)0)
#define QL_DMA_SETTLE() ((void)0)
#endif

// ---- LDS tiles -------------------------------------------------------------------------------
QL_DEV int swz_chunk(int chunk, int row) { return chunk ^ (((row >> 1) & 3) << 2 | (row & 1) * 3); }
QL_DEV int tile_off(int row, int chunk) { return row * kRowBytes + swz_chunk(chunk, row) * 16; }

// Transposing LDS read (ds_read_b64_tr_b16). Within each group of 16 lanes, lane i receives
// element i % 4 of the 8-B chunks addressed by lanes 4 j + i / 4, j = 0..3: with lane 4 j + c
// addressing row r_j, columns n0 + 4 c .. +3 of a row-major tile, lane i gets column n0 + i
// of rows r_0 .. r_3 (4 consecutive contraction values of an MFMA operand column).
QL_DEV uint2 read_tr(const char* p) {
  QL_DMA_READ(p);
  const v4i16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(p));
  return __builtin_bit_cast(uint2, r);
}

// Operand fragment (16 rows x 32 contraction) along the rows of a tile: lane holds row `row`,
// head-dim values 32 ks + 8 (lane / 16) .. +7.
QL_DEV uint4 frag_row(const char* __restrict__ t, int row, int ks, int fq) {
  QL_DMA_READ(t + tile_off(row, 4 * ks + fq));
  return *reinterpret_cast<const uint4*>(t + tile_off(row, 4 * ks + fq));
}

// Operand fragment whose contraction index runs over tile rows, read transposed: lane holds
// head-dim column c0 + lane % 16 at tile rows r0 + 4 (lane / 16) + j (positions 0..3) and
// r0 + 16 + 4 (lane / 16) + j (positions 4..7), the row order of two stacked C tiles, so it
// pairs with `pack_pair` operands. r0 is a multiple of 8.
QL_DEV uint4 frag_tr(const char* __restrict__ t, int r0, int c0, int fq, int fr) {
  const int row = r0 + 4 * fq + (fr >> 2);
  const int col = c0 + 4 * (fr & 3);
  const int off = tile_off(row, col >> 3) + (col & 4) * 2;
  const uint2 a = read_tr(t + off);
  const uint2 b = read_tr(t + off + 16 * kRowBytes);  // row + 16: same swizzle
  return make_uint4(a.x, a.y, b.x, b.y);
}

// Direct-to-LDS loader of one 64-row tile (rows row0 .. row0 + 63 of X, row stride ld
// elements; rows past S re-read row S - 1) by the 4 waves of a workgroup: load i of wave w
// fills tile rows 4p .. 4p + 3 with p = 4 i + w; lane l writes LDS bytes [16 l, 16 l + 16) of
// that 1 KiB span, i.e. row 4p + l / 16, physical chunk l % 16, which holds the logical chunk
// the swizzle maps there (an XOR is its own inverse). Row 4p + l / 16 has row & 15 =
// 4 w + l / 16 for every load, so the lane's byte offset from the span's first row is fixed:
// each load is a wave-uniform base (SGPRs) plus that offset.
// One direct-to-LDS load (16 B per lane from sbase + voff, lane l writing LDS bytes
// [lds + 16 l, lds + 16 l + 16)), written as inline assembly: the compiler's wait-count pass
// treats a pending direct-to-LDS load as an out-of-order LDS-counter event and then drains
// every LDS read (lgkmcnt(0)) before each product that uses one; with the load hidden from
// it, fragment reads are waited for in order, so reads issued ahead stay in flight. Nothing
// waits for these loads but wait_all_barrier, which every kernel runs before it reads a tile
// it loaded. (s_nop 4: the wait states a write of M0, or a VALU write of an address SGPR,
// needs before a vector memory load reads it; inline assembly gets no hazard padding.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is clobbered on purpose
QL_DEV void dma_b128(const char* sbase, uint32_t voff, char* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr_t)lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(m0)
               : "memory", "m0");
  QL_DMA_LOADED(lds);  // the 1 KiB this instruction fills: one span (tiles are 1-KiB aligned)
}
#pragma clang diagnostic pop

struct TileDma {
  uint32_t off;
  int rsub, wave;
  QL_DEV void init(int64_t ld, int wave_, int lane) {
    wave = wave_;
    rsub = lane >> 4;
    off = (uint32_t)rsub * (uint32_t)(ld * 2) +
          (uint32_t)(swz_chunk(lane & 15, 4 * wave + rsub) * 16);
  }
  QL_DEV void issue(const uint16_t* __restrict__ X, int64_t ld, int64_t row0, int64_t S,
                    char* __restrict__ tile) const {
    const int lane = threadIdx.x & 63;
    if (row0 + kRows <= S) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = 4 * i + wave;
        const char* base = reinterpret_cast<const char*>(X + (row0 + 4 * p) * ld);
        dma_b128(base, off, tile + p * 1024);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = 4 * i + wave;
        const int64_t gb = row0 + 4 * p;
        const int64_t base_row = gb < S ? gb : S - 1;
        const int64_t gr = gb + rsub < S ? gb + rsub : S - 1;
        const uint32_t o = (uint32_t)(gr - base_row) * (uint32_t)(ld * 2) +
                           (uint32_t)(swz_chunk(lane & 15, 4 * p + rsub) * 16);
        const char* base = reinterpret_cast<const char*>(X + base_row * ld);
        dma_b128(base, o, tile + p * 1024);
      }
    }
  }
};

// This thread's DMA and LDS writes are done, and every wave of the workgroup got here.
// (__syncthreads would also do, but inline asm keeps the compiler from adding its own waits.)
QL_DEV void wait_all_barrier() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  QL_DMA_SETTLE();
}

// This thread's ordinary global loads (the fragments a kernel keeps in registers across its
// block loop) have landed, said with a wait the compiler's wait-count pass sees. That pass
// cannot read wait_all_barrier's assembly: without this it counts those loads as pending in
// every block and waits for each before its first use there, and since vmcnt completes in
// issue order, each such wait also drains the next block's DMA issued since, so the prefetch
// no longer runs under the block's math.
QL_DEV void wait_vm_visible() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Index differences used by the masks, clamped into int range. The empty register barrier
// keeps the compiler from comparing the unclamped 64-bit value instead (an equivalent test,
// but two 64-bit compares per element of every masked block).
QL_DEV int clamp_rel(int64_t x) {
  int v = (int)(x < -4096 ? -4096 : x > 4096 ? 4096 : x);
  asm volatile("" : "+v"(v));
  return v;
}

struct AttnShape {
  int64_t B, HQ, HK, S;
  int64_t qs_b, qs_h, qs_s;  // element strides of q (last dim unit)
  int64_t ks_b, ks_h, ks_s;
  int64_t vs_b, vs_h, vs_s;
  int64_t os_b, os_h, os_s;
  float scale;
};

// =============================================================================================
// Forward. One workgroup per (b, hq, 128-row query block), heaviest (last) blocks first; wave
// w owns query rows 32 w .. +31. Per 64-key block:
//   S^T = K Q^T     K fragments from LDS, Q fragments in registers for the whole loop; a lane
//                   owns one query column (lane % 16) and 4 keys per 16-key tile
//   online softmax  per lane: block max over the lane's 16 keys plus two cross-lane steps, lazy
//                   rescaling of O (only when the max rises by more than kTau), the row sum
//                   kept per lane and combined once at the end
//   O^T += V^T P^T  V^T fragments by transposing reads, P^T straight from registers
template <int DT>
struct FwdState {
  uint4 qf[2][4];     // B operands: column q = 16 qt + lane % 16, d = 32 ds + 8 (lane / 16) ..
  f32x4_t o[2][8];    // [qt][dt]: rows d = 16 dt + 4 (lane / 16) + e, column q
  float m[2], l[2];
};

// `kl`, `vl`: this block's K and V tiles; `kn`, `vn`: the other stage, which the next block's
// DMA fills meanwhile (restrict keeps the compiler's wait-count pass from making these LDS
// reads wait for that DMA).
template <int DT>
QL_DEV void fwd_block(FwdState<DT>& st, const char* __restrict__ kl, const char* __restrict__ vl,
                      char* __restrict__ kn, char* __restrict__ vn, bool issue,
                      const TileDma& kdma, const TileDma& vdma, const uint16_t* __restrict__ kbase,
                      const uint16_t* __restrict__ vbase, int64_t ks_s, int64_t vs_s, int64_t key0,
                      int64_t q0, int64_t S, float sl2, int lane) {
  const int fr = lane & 15, fq = lane >> 4;
  if (issue) {
    kdma.issue(kbase, ks_s, key0 + kRows, S, kn);
    vdma.issue(vbase, vs_s, key0 + kRows, S, vn);
  }
  if (key0 > q0 + 31) return;  // every key of the block is after this wave's rows
  f32x4_t s[2][4];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) s[qt][kt] = zero4();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int ds = 0; ds < 4; ++ds)
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const uint4 kf = frag_row(kl, 16 * kt + fr, ds, fq);
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) s[qt][kt] = mfma<DT>(kf, st.qf[qt][ds], s[qt][kt]);
    }
  // 16 steps of 1 row read and 2 products; reads two steps ahead of their products
  __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
  for (int i = 0; i < 14; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
  __builtin_amdgcn_sched_barrier(0);
  // mask keys after the query row or past the end; block max per query column
  const bool need_mask = key0 + kRows - 1 > q0 || key0 + kRows > S;
  float bm[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    if (need_mask) {
      // key = key0 + 16 kt + 4 fq + e is kept iff 16 kt + e <= lim
      const int64_t q = q0 + 16 * qt + fr;
      const int64_t last = (q < S - 1 ? q : S - 1) - key0;
      const int lim = (int)(last < kRows ? last : kRows) - 4 * fq;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) s[qt][kt][e] = 16 * kt + e > lim ? -INFINITY : s[qt][kt][e];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) mx = fmaxf(mx, s[qt][kt][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    bm[qt] = mx * sl2;
  }
  const bool raise = bm[0] > st.m[0] + kTau || bm[1] > st.m[1] + kTau;
  if (__builtin_amdgcn_ballot_w64(raise)) {
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const float mn = fmaxf(st.m[qt], bm[qt]);
      const float alpha = __builtin_amdgcn_exp2f(st.m[qt] - mn);  // m = -inf: alpha = 0
      st.l[qt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) st.o[qt][dt] *= alpha;
      st.m[qt] = mn;
    }
  }
  uint4 pf[2][2];  // [ks][qt]
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float nm = -st.m[qt];
    float rs = 0.f;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qt][kt][e], sl2, nm));
        s[qt][kt][e] = p;
        rs += p;
      }
    st.l[qt] += rs;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) pf[ks][qt] = pack_pair<DT>(s[qt][2 * ks], s[qt][2 * ks + 1]);
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint4 vf = frag_tr(vl, 32 * ks, 16 * dt, fq, fr);
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) st.o[qt][dt] = mfma<DT>(vf, pf[ks][qt], st.o[qt][dt]);
    }
}

template <int DT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fwd_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                     const uint16_t* __restrict__ V, uint16_t* __restrict__ O,
                     float* __restrict__ lse, AttnShape sh, int n_qblocks) {
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTileBytes];  // [stage][K, V]
  QL_DMA_BEGIN();
  const int64_t BH = sh.B * sh.HQ;
  const int qb = n_qblocks - 1 - (int)(blockIdx.x / BH);  // heaviest blocks first
  const int64_t bh = blockIdx.x % BH;
  const int64_t b = bh / sh.HQ, hq = bh % sh.HQ;
  const int64_t hk = hq / (sh.HQ / sh.HK);
  const int64_t S = sh.S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int fr = lane & 15, fq = lane >> 4;
  const int64_t q0 = (int64_t)qb * BQ + 32 * wave;  // this wave's first query row

  const uint16_t* qbase = Q + b * sh.qs_b + hq * sh.qs_h;
  const uint16_t* kbase = K + b * sh.ks_b + hk * sh.ks_h;
  const uint16_t* vbase = V + b * sh.vs_b + hk * sh.vs_h;

  FwdState<DT> st;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t q = q0 + 16 * qt + fr;
    const int64_t qc = q < S ? q : S - 1;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
      st.qf[qt][ds] = *reinterpret_cast<const uint4*>(qbase + qc * sh.qs_s + 32 * ds + 8 * fq);
    st.m[qt] = -INFINITY;
    st.l[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) st.o[qt][dt] = zero4();
  }
  const float sl2 = sh.scale * kLog2e;
  const int64_t q_end = (int64_t)(qb + 1) * BQ;  // causal: keys < q_end
  const int64_t kv_end = q_end < S ? q_end : S;
  const int nkv = (int)((kv_end + kRows - 1) / kRows);

  TileDma kdma, vdma;
  kdma.init(sh.ks_s, wave, lane);
  vdma.init(sh.vs_s, wave, lane);
  kdma.issue(kbase, sh.ks_s, 0, S, smem);
  vdma.issue(vbase, sh.vs_s, 0, S, smem + kTileBytes);
  wait_vm_visible();  // the q fragments
  for (int j = 0; j < nkv; ++j) {
    // block j's tiles are in LDS, and every wave is past block j - 1, whose stage the DMA
    // issued in this step overwrites
    wait_all_barrier();
    char* cur = smem + (j & 1) * 2 * kTileBytes;
    char* nxt = smem + ((j + 1) & 1) * 2 * kTileBytes;
    fwd_block<DT>(st, cur, cur + kTileBytes, nxt, nxt + kTileBytes, j + 1 < nkv, kdma, vdma,
                  kbase, vbase, sh.ks_s, sh.vs_s, (int64_t)j * kRows, q0, S, sl2, lane);
  }

  // O = O^T / l, lse = (m + log2 l) ln 2 (natural log of sum exp(scale * s))
  uint16_t* obase = O + b * sh.os_b + hq * sh.os_h;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    float l = st.l[qt];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int64_t q = q0 + 16 * qt + fr;
    if (q >= S) continue;
    const float inv = 1.0f / l;
    uint16_t* orow = obase + q * sh.os_s;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f32x4_t v = st.o[qt][dt] * inv;
      *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * fq) =
          make_uint2(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]));
    }
    if (fq == 0 && lse) lse[bh * S + q] = (st.m[qt] + log2f(l)) * kLn2;
  }
}

// =============================================================================================
// Backward.
struct BwdShape {
  int64_t B, HQ, HK, S;
  int64_t qs_b, qs_h, qs_s, ks_b, ks_h, ks_s, vs_b, vs_h, vs_s;
  int64_t os_b, os_h, os_s;   // o and do (same layout)
  int64_t dq_b, dq_h, dq_s;   // dq
  int64_t dk_b, dk_h, dk_s;   // dk and dv (same layout)
  float scale;
};

// ---- dK, dV: one workgroup per (b, hq, 64-key block), heaviest (first) key blocks first; wave
// w owns keys 16 w .. +15 of the block. Per 64-row query block at or below the diagonal:
//   S = Q K^T, dP = dO V^T      Q, dO row fragments from LDS; K, V fragments in registers
//   P = exp2(S scale log2e - lse log2e), dS = P (dP - Delta)
//   dV^T += dO^T P, dK^T += Q^T dS    dO^T, Q^T by transposing reads; P, dS from registers
// With several query heads per kv head, each head's dK, dV go to partials in the input type
// that attn_bwd_reduce sums in fp32 in head order; otherwise the kernel writes the 16-bit
// gradients itself. (The reference's grouped-query path rounds each repeated head's gradient
// to the input type too before the repeat's backward sums them: 16-bit partials add no rounding
// it does not have, and halve the partials' traffic against fp32 ones.)
constexpr int kBwdStage = 2 * kTileBytes + 512;  // Q tile, dO tile, lse2 [64], delta [64]

template <int DT>
struct DkdvState {
  uint4 kf[4], vf[4];      // B operands: column key lane % 16, d = 32 ds + 8 (lane / 16) .. +7
  f32x4_t dv[8], dk[8];    // [dt]: rows d = 16 dt + 4 (lane / 16) + e, column key
};

template <int DT>
QL_DEV void dkdv_block(DkdvState<DT>& st, const char* __restrict__ cur, char* __restrict__ nxt,
                       bool issue, const TileDma& qdma, const TileDma& odma,
                       const uint16_t* __restrict__ qbase, const uint16_t* __restrict__ obase,
                       int64_t qs_s, int64_t os_s, int64_t qrow0, int64_t S, bool need_mask,
                       int kq_rel, int qlim, float sl2, int lane) {
  const int fr = lane & 15, fq = lane >> 4;
  if (issue) {
    qdma.issue(qbase, qs_s, qrow0 + kRows, S, nxt);
    odma.issue(obase, os_s, qrow0 + kRows, S, nxt + kTileBytes);
  }
  const char* q_l = cur;
  const char* do_l = cur + kTileBytes;
  const float* lse2 = reinterpret_cast<const float*>(cur + 2 * kTileBytes);
  const float* dlt = lse2 + kRows;
  f32x4_t sp[4], dp[4];  // [qt]: rows q = 16 qt + 4 (lane / 16) + e, column key
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) sp[qt] = dp[qt] = zero4();
#pragma unroll
  for (int ds = 0; ds < 4; ++ds)
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
      const int row = 16 * qt + fr;
      sp[qt] = mfma<DT>(frag_row(q_l, row, ds, fq), st.kf[ds], sp[qt]);
      dp[qt] = mfma<DT>(frag_row(do_l, row, ds, fq), st.vf[ds], dp[qt]);
    }
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    const float4 l4 = *reinterpret_cast<const float4*>(lse2 + 16 * qt + 4 * fq);
    const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      sp[qt][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sp[qt][e], sl2, -lv[e]));
  }
  // Only the diagonal block and a block past the end have masked entries: a wave-uniform
  // branch, so the other blocks skip the tests. key - q = kq_rel - 16 qt - e; rows at or past
  // the end: 16 qt + e >= qlim.
  if (__builtin_expect(need_mask, 0)) {
#pragma unroll
    for (int qt = 0; qt < 4; ++qt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (kq_rel - 16 * qt - e > 0 || 16 * qt + e >= qlim) sp[qt][e] = 0.f;
  }
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    const float4 d4 = *reinterpret_cast<const float4*>(dlt + 16 * qt + 4 * fq);
    const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) dp[qt][e] = sp[qt][e] * (dp[qt][e] - dv[e]);
  }
  uint4 pb[2], sb[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    pb[ks] = pack_pair<DT>(sp[2 * ks], sp[2 * ks + 1]);
    sb[ks] = pack_pair<DT>(dp[2 * ks], dp[2 * ks + 1]);
  }
  __builtin_amdgcn_sched_barrier(0);
  // 16 steps (ks, dt) of 4 transposing reads and 2 products. The reads run two steps ahead
  // of their products, so a product waits on reads issued two steps earlier rather than on
  // the latest one (left to itself the scheduler, short of registers, put each read right
  // before its product and waited for it).
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int ks = i >> 3, dt = i & 7;
    st.dv[dt] = mfma<DT>(frag_tr(do_l, 32 * ks, 16 * dt, fq, fr), pb[ks], st.dv[dt]);
    st.dk[dt] = mfma<DT>(frag_tr(q_l, 32 * ks, 16 * dt, fq, fr), sb[ks], st.dk[dt]);
  }
  __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
  for (int i = 0; i < 14; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
  __builtin_amdgcn_sched_barrier(0);
}

template <int DT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_bwd_dkdv(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                   const uint16_t* __restrict__ V, const uint16_t* __restrict__ dO,
                   const float* __restrict__ lse, const float* __restrict__ delta,
                   uint16_t* __restrict__ dK, uint16_t* __restrict__ dV,
                   uint16_t* __restrict__ pk, uint16_t* __restrict__ pv, BwdShape sh,
                   int n_kblocks) {
  __shared__ __attribute__((aligned(1024))) char smem[2 * kBwdStage];
  QL_DMA_BEGIN();
  const int64_t BH = sh.B * sh.HQ;
  const int kb = (int)(blockIdx.x / BH);  // heaviest (first) key blocks first
  const int64_t bh = blockIdx.x % BH;
  const int64_t b = bh / sh.HQ, hq = bh % sh.HQ;
  const int64_t hk = hq / (sh.HQ / sh.HK);
  const int64_t S = sh.S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int fr = lane & 15, fq = lane >> 4;
  const int64_t key0w = (int64_t)kb * kRows + 16 * wave;  // this wave's first key
  const float sl2 = sh.scale * kLog2e;

  DkdvState<DT> st;
  const uint16_t* kbase = K + b * sh.ks_b + hk * sh.ks_h;
  const uint16_t* vbase = V + b * sh.vs_b + hk * sh.vs_h;
  {
    const int64_t key = key0w + fr;
    const int64_t kc = key < S ? key : S - 1;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      st.kf[ds] = *reinterpret_cast<const uint4*>(kbase + kc * sh.ks_s + 32 * ds + 8 * fq);
      st.vf[ds] = *reinterpret_cast<const uint4*>(vbase + kc * sh.vs_s + 32 * ds + 8 * fq);
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) st.dv[dt] = st.dk[dt] = zero4();
  }

  const uint16_t* qbase = Q + b * sh.qs_b + hq * sh.qs_h;
  const uint16_t* obase = dO + b * sh.os_b + hq * sh.os_h;
  const float* lse_row = lse + bh * S;
  const float* dl_row = delta + bh * S;
  const int n_qb = n_kblocks;  // 64-row query blocks
  TileDma qdma, odma;
  qdma.init(sh.qs_s, wave, lane);
  odma.init(sh.os_s, wave, lane);
  // lse * log2e and Delta of a query block: thread t < 128 stages row t & 63 of one of them.
  // The load goes out before the block's math and the lse is scaled only where it is staged,
  // after that math, so no wave waits on the load's latency inside the block.
  const int t = threadIdx.x;
  auto row_stat = [&](int qb) -> float {
    const int64_t q = (int64_t)qb * kRows + (t & 63);
    const int64_t qc = q < S ? q : S - 1;
    return t < 64 ? lse_row[qc] : dl_row[qc];
  };
  auto stage_stat = [&](char* stage, float v) {
    reinterpret_cast<float*>(stage + 2 * kTileBytes)[t] = t < 64 ? v * kLog2e : v;
  };
  qdma.issue(qbase, sh.qs_s, (int64_t)kb * kRows, S, smem);
  odma.issue(obase, sh.os_s, (int64_t)kb * kRows, S, smem + kTileBytes);
  if (t < 128) stage_stat(smem, row_stat(kb));
  wait_vm_visible();  // the k and v fragments
  for (int qb = kb; qb < n_qb; ++qb) {
    wait_all_barrier();
    const int it = qb - kb;
    char* cur = smem + (it & 1) * kBwdStage;
    char* nxt = smem + ((it + 1) & 1) * kBwdStage;
    const bool more = qb + 1 < n_qb;
    float stat = 0.f;
    if (more && t < 128) stat = row_stat(qb + 1);
    const int64_t qrow0 = (int64_t)qb * kRows;
    const bool need_mask = qb == kb || qrow0 + kRows > S;
    const int kq_rel = clamp_rel(key0w + fr - (qrow0 + 4 * fq));
    const int qlim = clamp_rel(S - (qrow0 + 4 * fq));
    dkdv_block<DT>(st, cur, nxt, more, qdma, odma, qbase, obase, sh.qs_s, sh.os_s, qrow0, S,
                   need_mask, kq_rel, qlim, sl2, lane);
    if (more && t < 128) stage_stat(nxt, stat);
  }

  const int64_t key = key0w + fr;
  if (key >= S) return;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    const f32x4_t v = st.dv[dt];
    const f32x4_t k4 = st.dk[dt] * sh.scale;
    const int d = 16 * dt + 4 * fq;
    if (pk) {
      const int64_t row = (bh * S + key) * HD + d;
      *reinterpret_cast<uint2*>(pv + row) = make_uint2(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]));
      *reinterpret_cast<uint2*>(pk + row) =
          make_uint2(pack2<DT>(k4[0], k4[1]), pack2<DT>(k4[2], k4[3]));
    } else {
      uint16_t* dvp = dV + b * sh.dk_b + hk * sh.dk_h + key * sh.dk_s + d;
      uint16_t* dkp = dK + b * sh.dk_b + hk * sh.dk_h + key * sh.dk_s + d;
      *reinterpret_cast<uint2*>(dvp) = make_uint2(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]));
      *reinterpret_cast<uint2*>(dkp) = make_uint2(pack2<DT>(k4[0], k4[1]), pack2<DT>(k4[2], k4[3]));
    }
  }
}

// dK[b, s, hk] = sum_g pk[b, hk G + g, s], dV likewise, in fp32 in head order (one thread per
// 8 d).
template <int DT>
__global__ __launch_bounds__(256) void attn_bwd_reduce(const uint16_t* __restrict__ pk,
                                                        const uint16_t* __restrict__ pv,
                                                        uint16_t* __restrict__ dK,
                                                        uint16_t* __restrict__ dV, BwdShape sh) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = sh.B * sh.HK * sh.S * (HD / 8);
  if (idx >= total) return;
  const int part = (int)(idx & 15);
  const int64_t r = idx >> 4;  // (b, hk, s)
  const int64_t s = r % sh.S, bhk = r / sh.S;
  const int64_t b = bhk / sh.HK, hk = bhk % sh.HK;
  const int64_t G = sh.HQ / sh.HK;
  float ak[8] = {}, av[8] = {};
  for (int64_t g = 0; g < G; ++g) {
    const int64_t off = ((b * sh.HQ + hk * G + g) * sh.S + s) * HD + 8 * part;
    float k8[8], v8[8];
    Vec8<DT>::load(pk + off, k8);
    Vec8<DT>::load(pv + off, v8);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ak[j] += k8[j];
      av[j] += v8[j];
    }
  }
  const int64_t o = b * sh.dk_b + hk * sh.dk_h + s * sh.dk_s + 8 * part;
  Vec8<DT>::store(dK + o, ak);
  Vec8<DT>::store(dV + o, av);
}

// ---- dQ: one workgroup per (b, hq, 128-row query block), heaviest first; wave w owns rows
// 32 w .. +31. Per 64-key block, in two 32-key halves:
//   S^T = K Q^T, dP^T = V dO^T    K, V row fragments from LDS; Q, dO fragments in registers
//   dS^T = P^T (dP^T - Delta)
//   dQ^T += K^T dS^T               K^T by transposing reads; dS^T from registers
template <int DT>
struct DqState {
  uint4 qf[2][4], df[2][4];  // B operands: column q = 16 qt + lane % 16, d = 32 ds + 8 (lane/16)
  f32x4_t dq[2][8];          // [qt][dt]: rows d = 16 dt + 4 (lane / 16) + e, column q
  float l2[2], dl[2];        // lse * log2e and Delta of the lane's query columns
};

template <int DT>
QL_DEV void dq_block(DqState<DT>& st, const char* __restrict__ kl, const char* __restrict__ vl,
                     char* __restrict__ kn, char* __restrict__ vn, bool issue, const TileDma& kdma,
                     const TileDma& vdma, const uint16_t* __restrict__ kbase,
                     const uint16_t* __restrict__ vbase, int64_t ks_s, int64_t vs_s, int64_t key0,
                     int64_t q0, int64_t S, float sl2, int lane) {
  const int fr = lane & 15, fq = lane >> 4;
  if (issue) {
    kdma.issue(kbase, ks_s, key0 + kRows, S, kn);
    vdma.issue(vbase, vs_s, key0 + kRows, S, vn);
  }
  if (key0 > q0 + 31) return;
  const bool need_mask = key0 + kRows - 1 > q0 || key0 + kRows > S;
  // key - q = kq_rel + 32 h + 16 kk + e - 16 qt; keys at or past the end: 32 h + 16 kk + e >= klim
  const int kq_rel = clamp_rel(key0 + 4 * fq - (q0 + fr));
  const int klim = clamp_rel(S - key0 - 4 * fq);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    f32x4_t sp[2][2], dp[2][2];  // [qt][kk]: rows key 32 h + 16 kk + 4 (lane/16) + e, column q
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) sp[qt][kk] = dp[qt][kk] = zero4();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int row = 32 * h + 16 * kk + fr;
        const uint4 ka = frag_row(kl, row, ds, fq);
        const uint4 va = frag_row(vl, row, ds, fq);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          sp[qt][kk] = mfma<DT>(ka, st.qf[qt][ds], sp[qt][kk]);
          dp[qt][kk] = mfma<DT>(va, st.df[qt][ds], dp[qt][kk]);
        }
      }
    // 8 steps of 2 row reads and 4 products; reads two steps ahead of their products
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          sp[qt][kk][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sp[qt][kk][e], sl2, -st.l2[qt]));
    if (__builtin_expect(need_mask, 0)) {  // wave-uniform: the diagonal and end blocks only
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int rel = 32 * h + 16 * kk + e;
            if (kq_rel + rel - 16 * qt > 0 || rel >= klim) sp[qt][kk][e] = 0.f;
          }
    }
    uint4 sb[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int e = 0; e < 4; ++e) dp[qt][kk][e] = sp[qt][kk][e] * (dp[qt][kk][e] - st.dl[qt]);
      sb[qt] = pack_pair<DT>(dp[qt][0], dp[qt][1]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint4 ka = frag_tr(kl, 32 * h, 16 * dt, fq, fr);
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) st.dq[qt][dt] = mfma<DT>(ka, sb[qt], st.dq[qt][dt]);
    }
    // 8 steps of 2 transposing reads and 2 products; reads two steps ahead
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_bwd_dq(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                 const uint16_t* __restrict__ V, const uint16_t* __restrict__ O,
                 const uint16_t* __restrict__ dO, const float* __restrict__ lse,
                 float* __restrict__ delta, uint16_t* __restrict__ dQ, BwdShape sh,
                 int n_qblocks) {
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTileBytes];  // [stage][K, V]
  QL_DMA_BEGIN();
  const int64_t BH = sh.B * sh.HQ;
  const int qb = n_qblocks - 1 - (int)(blockIdx.x / BH);  // heaviest blocks first
  const int64_t bh = blockIdx.x % BH;
  const int64_t b = bh / sh.HQ, hq = bh % sh.HQ;
  const int64_t hk = hq / (sh.HQ / sh.HK);
  const int64_t S = sh.S;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int fr = lane & 15, fq = lane >> 4;
  const int64_t q0 = (int64_t)qb * BQ + 32 * wave;
  const float sl2 = sh.scale * kLog2e;

  DqState<DT> st;
  const uint16_t* qbase = Q + b * sh.qs_b + hq * sh.qs_h;
  const uint16_t* dobase = dO + b * sh.os_b + hq * sh.os_h;
  const uint16_t* obase = O + b * sh.os_b + hq * sh.os_h;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t q = q0 + 16 * qt + fr;
    const int64_t qc = q < S ? q : S - 1;
    uint4 of[4];
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      st.qf[qt][ds] = *reinterpret_cast<const uint4*>(qbase + qc * sh.qs_s + 32 * ds + 8 * fq);
      st.df[qt][ds] = *reinterpret_cast<const uint4*>(dobase + qc * sh.os_s + 32 * ds + 8 * fq);
      of[ds] = *reinterpret_cast<const uint4*>(obase + qc * sh.os_s + 32 * ds + 8 * fq);
    }
    st.l2[qt] = lse[bh * S + qc] * kLog2e;
    // Delta = rowsum(dO * O) of this lane's row (the FlashAttention-2 backward's D), in a fixed
    // order: 16 parts of 8 consecutive d (part p = 4 ds + fq holds d = 8 p .. 8 p + 7, an fma
    // chain), combined by a butterfly over p ^ 8, p ^ 4, p ^ 2, p ^ 1; the first two flip ds
    // (within this lane), the last two fq (lanes ^ 32 and ^ 16), so every lane of the row ends
    // with the same value. The dQ kernel runs first and stores it for the dK/dV kernel.
    float part[4];
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      float o8[8], d8[8];
      Vec8<DT>::unpack(of[ds], o8);
      Vec8<DT>::unpack(st.df[qt][ds], d8);
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(o8[j], d8[j], acc);
      part[ds] = acc;
    }
    float dl = (part[0] + part[2]) + (part[1] + part[3]);
    dl += __shfl_xor(dl, 32, 64);
    dl += __shfl_xor(dl, 16, 64);
    st.dl[qt] = dl;
    if (fq == 0 && q < S) delta[bh * S + q] = dl;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) st.dq[qt][dt] = zero4();
  }
  const int64_t q_end = (int64_t)(qb + 1) * BQ;
  const int64_t kv_end = q_end < S ? q_end : S;
  const int nkv = (int)((kv_end + kRows - 1) / kRows);
  const uint16_t* kbase = K + b * sh.ks_b + hk * sh.ks_h;
  const uint16_t* vbase = V + b * sh.vs_b + hk * sh.vs_h;
  TileDma kdma, vdma;
  kdma.init(sh.ks_s, wave, lane);
  vdma.init(sh.vs_s, wave, lane);
  kdma.issue(kbase, sh.ks_s, 0, S, smem);
  vdma.issue(vbase, sh.vs_s, 0, S, smem + kTileBytes);
  wait_vm_visible();  // the q and dO fragments and lse (Delta is computed above)
  for (int j = 0; j < nkv; ++j) {
    wait_all_barrier();
    char* cur = smem + (j & 1) * 2 * kTileBytes;
    char* nxt = smem + ((j + 1) & 1) * 2 * kTileBytes;
    dq_block<DT>(st, cur, cur + kTileBytes, nxt, nxt + kTileBytes, j + 1 < nkv, kdma, vdma,
                 kbase, vbase, sh.ks_s, sh.vs_s, (int64_t)j * kRows, q0, S, sl2, lane);
  }
  uint16_t* dqb = dQ + b * sh.dq_b + hq * sh.dq_h;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t q = q0 + 16 * qt + fr;
    if (q >= S) continue;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f32x4_t v = st.dq[qt][dt] * sh.scale;
      *reinterpret_cast<uint2*>(dqb + q * sh.dq_s + 16 * dt + 4 * fq) =
          make_uint2(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]));
    }
  }
}

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

}  // namespace

extern "C" int qlora_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                              int dtype, int64_t B, int64_t HQ, int64_t HK, int64_t S, int64_t D,
                              const int64_t* q_strides, const int64_t* k_strides,
                              const int64_t* v_strides, const int64_t* o_strides, float scale,
                              ql_stream_t stream) {
  if (B < 0 || HQ <= 0 || HK <= 0 || S < 0 || HQ % HK) return QL_EINVAL;
  if (D != HD) return QL_ESHAPE;
  if (dtype != QL_BF16 && dtype != QL_F16) return QL_EDTYPE;
  if (B == 0 || S == 0) return QL_OK;
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return QL_EINVAL;
  AttnShape sh;
  sh.B = B; sh.HQ = HQ; sh.HK = HK; sh.S = S; sh.scale = scale;
  sh.qs_b = q_strides[0]; sh.qs_h = q_strides[1]; sh.qs_s = q_strides[2];
  sh.ks_b = k_strides[0]; sh.ks_h = k_strides[1]; sh.ks_s = k_strides[2];
  sh.vs_b = v_strides[0]; sh.vs_h = v_strides[1]; sh.vs_s = v_strides[2];
  sh.os_b = o_strides[0]; sh.os_h = o_strides[1]; sh.os_s = o_strides[2];
  // every row start must be 16-B aligned for the vector loads and 8-B stores
  const int64_t strides[12] = {sh.qs_b, sh.qs_h, sh.qs_s, sh.ks_b, sh.ks_h, sh.ks_s,
                               sh.vs_b, sh.vs_h, sh.vs_s, sh.os_b, sh.os_h, sh.os_s};
  for (int64_t st : strides)
    if (st % 8) return QL_EALIGN;
  if (!ql_aligned(q, 16) || !ql_aligned(k, 16) || !ql_aligned(v, 16) || !ql_aligned(o, 16))
    return QL_EALIGN;
  const int n_qblocks = (int)((S + BQ - 1) / BQ);
  const int64_t grid = B * HQ * n_qblocks;
  if (grid > INT32_MAX) return QL_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == QL_BF16)
    hipLaunchKernelGGL((attn_fwd_kernel<QL_BF16>), dim3((unsigned)grid), dim3(kThreads), 0, s,
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o,
                       lse, sh, n_qblocks);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<QL_F16>), dim3((unsigned)grid), dim3(kThreads), 0, s,
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o,
                       lse, sh, n_qblocks);
  return ql_launch_status();
}

extern "C" int64_t qlora_attn_bwd_workspace_size(int64_t B, int64_t HQ, int64_t HK, int64_t S) {
  if (B <= 0 || HQ <= 0 || HK <= 0 || S <= 0 || HQ % HK) return 0;
  int64_t bytes = align256(B * HQ * S * (int64_t)sizeof(float));   // Delta
  if (HQ != HK) bytes += 2 * align256(B * HQ * S * HD * (int64_t)sizeof(uint16_t));  // partials
  return bytes;
}

extern "C" int qlora_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                              const void* d_o, const float* lse, void* dq, void* dk, void* dv,
                              int dtype, int64_t B, int64_t HQ, int64_t HK, int64_t S, int64_t D,
                              const int64_t* q_strides, const int64_t* k_strides,
                              const int64_t* v_strides, const int64_t* o_strides,
                              const int64_t* dq_strides, const int64_t* dkv_strides, float scale,
                              void* workspace, int64_t workspace_bytes, ql_stream_t stream) {
  if (B < 0 || HQ <= 0 || HK <= 0 || S < 0 || HQ % HK) return QL_EINVAL;
  if (D != HD) return QL_ESHAPE;
  if (dtype != QL_BF16 && dtype != QL_F16) return QL_EDTYPE;
  if (B == 0 || S == 0) return QL_OK;
  if (!q || !k || !v || !o || !d_o || !lse || !dq || !dk || !dv || !q_strides || !k_strides ||
      !v_strides || !o_strides || !dq_strides || !dkv_strides)
    return QL_EINVAL;
  if (workspace_bytes < qlora_attn_bwd_workspace_size(B, HQ, HK, S) || !workspace ||
      !ql_aligned(workspace, 16))
    return QL_EINVAL;
  BwdShape sh;
  sh.B = B; sh.HQ = HQ; sh.HK = HK; sh.S = S; sh.scale = scale;
  sh.qs_b = q_strides[0]; sh.qs_h = q_strides[1]; sh.qs_s = q_strides[2];
  sh.ks_b = k_strides[0]; sh.ks_h = k_strides[1]; sh.ks_s = k_strides[2];
  sh.vs_b = v_strides[0]; sh.vs_h = v_strides[1]; sh.vs_s = v_strides[2];
  sh.os_b = o_strides[0]; sh.os_h = o_strides[1]; sh.os_s = o_strides[2];
  sh.dq_b = dq_strides[0]; sh.dq_h = dq_strides[1]; sh.dq_s = dq_strides[2];
  sh.dk_b = dkv_strides[0]; sh.dk_h = dkv_strides[1]; sh.dk_s = dkv_strides[2];
  const int64_t strides[18] = {sh.qs_b, sh.qs_h, sh.qs_s, sh.ks_b, sh.ks_h, sh.ks_s,
                               sh.vs_b, sh.vs_h, sh.vs_s, sh.os_b, sh.os_h, sh.os_s,
                               sh.dq_b, sh.dq_h, sh.dq_s, sh.dk_b, sh.dk_h, sh.dk_s};
  for (int64_t st : strides)
    if (st % 8) return QL_EALIGN;
  const void* ptrs[9] = {q, k, v, o, d_o, dq, dk, dv, lse};
  for (const void* p : ptrs)
    if (!ql_aligned(p, 16)) return QL_EALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  float* delta = reinterpret_cast<float*>(ws);
  uint16_t* pk = nullptr;
  uint16_t* pv = nullptr;
  if (HQ != HK) {
    const int64_t part_bytes = align256(B * HQ * S * HD * (int64_t)sizeof(uint16_t));
    pk = reinterpret_cast<uint16_t*>(ws + align256(B * HQ * S * (int64_t)sizeof(float)));
    pv = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(pk) + part_bytes);
  }
  const int n_kblocks = (int)((S + kRows - 1) / kRows);
  const int n_qblocks = (int)((S + BQ - 1) / BQ);
  if (B * HQ * n_kblocks > INT32_MAX || B * HQ * n_qblocks > INT32_MAX ||
      (B * HK * S * 16 + 255) / 256 > INT32_MAX)
    return QL_EINVAL;
#define QL_ATTN_BWD(DTC)                                                                          \
  do {                                                                                            \
    hipLaunchKernelGGL((attn_bwd_dq<DTC>), dim3((unsigned)(B * HQ * n_qblocks)), dim3(kThreads),  \
                       0, s, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,          \
                       (const uint16_t*)o, (const uint16_t*)d_o, lse, delta, (uint16_t*)dq, sh,   \
                       n_qblocks);                                                                \
    hipLaunchKernelGGL((attn_bwd_dkdv<DTC>), dim3((unsigned)(B * HQ * n_kblocks)), dim3(kThreads), \
                       0, s, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,          \
                       (const uint16_t*)d_o, lse, delta, (uint16_t*)dk, (uint16_t*)dv, pk, pv,    \
                       sh, n_kblocks);                                                            \
    if (pk)                                                                                       \
      hipLaunchKernelGGL((attn_bwd_reduce<DTC>), dim3((unsigned)((B * HK * S * 16 + 255) / 256)), \
                         dim3(256), 0, s, pk, pv, (uint16_t*)dk, (uint16_t*)dv, sh);              \
  } while (0)
  if (dtype == QL_BF16) QL_ATTN_BWD(QL_BF16);
  else QL_ATTN_BWD(QL_F16);
#undef QL_ATTN_BWD
  return ql_launch_status();
}

#ifdef QL_DMA_CHECK
// Debug builds only: the violations the ordering check counted since the last reset.
extern "C" int qlora_debug_dma_violations(unsigned long long* out, int reset) {
  if (hipMemcpyFromSymbol(out, HIP_SYMBOL(g_dma_violations), sizeof(*out)) != hipSuccess)
    return QL_EINVAL;
  if (reset) {
    const unsigned long long zero = 0;
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_dma_violations), &zero, sizeof(zero)) != hipSuccess)
      return QL_EINVAL;
  }
  return QL_OK;
}
#endif
