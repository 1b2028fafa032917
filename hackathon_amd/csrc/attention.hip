// Causal flash attention (forward) for the QLoRA step's attention, on CDNA4 matrix cores.
//
// The reference step runs attention through torch's scaled_dot_product_attention
// (transformers/models/qwen2/modeling_qwen2.py:220, the SDPA path of Qwen2Attention); this is
// the native replacement: O = softmax(Q K^T * scale, causal) V with grouped-query heads, bf16
// in and out, fp32 accumulation and softmax, and the row log-sum-exp kept for the backward.
//
// One workgroup (4 waves) per (batch, query head, 128-row query block); wave w owns query
// rows 32w .. 32w+31 of the block. Per 64-key block:
//   S^T = K Q^T      v_mfma_f32_16x16x32: K fragments from LDS ([key][d], 16-B chunks XOR-
//                    swizzled by key & 7), Q fragments held in registers for the whole loop.
//                    A lane ends up owning one query column (lane % 16) and 4 keys per 16-key
//                    tile, so the online softmax is per lane plus two cross-lane steps.
//   P = exp2(S log2e * scale - m)   online max / sum in fp32 (masked keys: -inf)
//   O^T += V^T P^T   the P^T register tile is itself the B operand (a 32-key step is two
//                    16-key tiles; the key order inside an MFMA step is a permutation, used
//                    identically for V^T); V^T comes from LDS ([d][key], 8-B units XOR-
//                    swizzled by d & 15), written there through an in-register 8 x 8 transpose.
// The next key block is loaded into registers while the current one is multiplied.
// Requires head_dim = 128; any sequence length (rows and keys past the end are masked).
#include "ql_vec.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

constexpr int HD = 128;        // head dim
constexpr int BQ = 128;        // query rows per workgroup
constexpr int BKV = 64;        // keys per block
constexpr int kThreads = 256;
constexpr int kKRow = HD * 2;  // bytes per K row in LDS (256)
constexpr int kVRow = BKV * 2; // bytes per V^T row in LDS (128)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

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

// 8 x 8 transpose of 16-bit values: in[i] = row i as 4 words (column pairs) -> out[t] = column t.
QL_DEV void transpose8x8(const uint4 (&in)[8], uint4 (&out)[8]) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint4& r0 = in[2 * p];
      const uint4& r1 = in[2 * p + 1];
      const int q = t >> 1;
      const uint32_t a = q == 0 ? r0.x : q == 1 ? r0.y : q == 2 ? r0.z : r0.w;
      const uint32_t b = q == 0 ? r1.x : q == 1 ? r1.y : q == 2 ? r1.z : r1.w;
      w[p] = (t & 1) ? __builtin_amdgcn_perm(b, a, 0x07060302u) : __builtin_amdgcn_perm(b, a, 0x05040100u);
    }
    out[t] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

struct AttnShape {
  int64_t B, HQ, HK, S;
  int64_t qs_b, qs_h, qs_s;  // element strides of q (last dim unit)
  int64_t ks_b, ks_h, ks_s;
  int64_t vs_b, vs_h, vs_s;
  int64_t os_b, os_h, os_s;
  float scale;
};

// Staging registers of one 64-key block for this thread: threads 0..127 hold 8 16-B chunks of
// K (key rows), threads 128..255 an 8 (key) x 8 (d) block of V.
struct KVStage {
  uint4 r[8];
};

QL_DEV void load_kv(KVStage& st, const uint16_t* __restrict__ kbase, int64_t ks_s,
                    const uint16_t* __restrict__ vbase, int64_t vs_s, int64_t key0, int64_t S) {
  const int t = threadIdx.x;
  if (t < 128) {
    // K: 64 rows x 16 chunks = 1024 chunks; chunk id c = t + 128 i: row c / 16, chunk c % 16
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = t + 128 * i;
      const int64_t key = key0 + (c >> 4);
      const int64_t kc = key < S ? key : S - 1;
      st.r[i] = *reinterpret_cast<const uint4*>(kbase + kc * ks_s + (c & 15) * 8);
    }
  } else {
    // V: 8 key groups x 16 d groups; thread u = t - 128 takes key group u / 16, d group u % 16
    const int u = t - 128;
    const int64_t kg = key0 + 8 * (u >> 4);
    const int dg = 8 * (u & 15);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t key = kg + i;
      const int64_t kc = key < S ? key : S - 1;
      st.r[i] = *reinterpret_cast<const uint4*>(vbase + kc * vs_s + dg);
    }
  }
}

// Write a staged block into LDS: K rows swizzled by 16-B chunk, V transposed into [d][key]
// rows swizzled by 8-B unit.
QL_DEV void store_kv(const KVStage& st, char* __restrict__ kl, char* __restrict__ vl) {
  const int t = threadIdx.x;
  if (t < 128) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = t + 128 * i;
      const int row = c >> 4, ch = c & 15;
      const int phys = ch ^ (row & 7);
      *reinterpret_cast<uint4*>(kl + row * kKRow + phys * 16) = st.r[i];
    }
  } else {
    const int u = t - 128;
    const int k0 = 8 * (u >> 4);
    const int d0 = 8 * (u & 15);
    uint4 tr[8];
    transpose8x8(st.r, tr);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int d = d0 + j;
      const int u0 = (k0 >> 2) ^ (d & 15), u1 = ((k0 >> 2) + 1) ^ (d & 15);
      *reinterpret_cast<uint2*>(vl + d * kVRow + u0 * 8) = make_uint2(tr[j].x, tr[j].y);
      *reinterpret_cast<uint2*>(vl + d * kVRow + u1 * 8) = make_uint2(tr[j].z, tr[j].w);
    }
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, float* __restrict__ lse, AttnShape sh, int n_qblocks) {
  __shared__ __attribute__((aligned(16))) char k_lds[2][BKV * kKRow];
  __shared__ __attribute__((aligned(16))) char v_lds[2][HD * kVRow];
  // heaviest (last) query blocks first
  const int qb = n_qblocks - 1 - (int)(blockIdx.x % n_qblocks);
  const int64_t bh = blockIdx.x / n_qblocks;
  const int64_t b = bh / sh.HQ, hq = bh % sh.HQ;
  const int64_t hk = hq / (sh.HQ / sh.HK);
  const int64_t S = sh.S;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int fr = lane & 15, fq = lane >> 4;
  const int64_t q0 = (int64_t)qb * BQ + 32 * wave;  // this wave's first query row

  const uint16_t* qbase = Q + b * sh.qs_b + hq * sh.qs_h;
  const uint16_t* kbase = K + b * sh.ks_b + hk * sh.ks_h;
  const uint16_t* vbase = V + b * sh.vs_b + hk * sh.vs_h;

  // Q fragments (B operand: column q = lane % 16, d = 32 ds + 8 (lane / 16) .. +7)
  uint4 qf[2][4];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t q = q0 + 16 * qt + fr;
    const int64_t qc = q < S ? q : S - 1;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
      qf[qt][ds] = *reinterpret_cast<const uint4*>(qbase + qc * sh.qs_s + 32 * ds + 8 * fq);
  }

  const float sl2 = sh.scale * kLog2e;
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
  f32x4_t o[2][8];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[qt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int64_t q_end = (int64_t)(qb + 1) * BQ;              // causal: keys < q_end
  const int64_t kv_end = q_end < S ? q_end : S;
  const int nkv = (int)((kv_end + BKV - 1) / BKV);

  KVStage st;
  load_kv(st, kbase, sh.ks_s, vbase, sh.vs_s, 0, S);
  store_kv(st, k_lds[0], v_lds[0]);
  __syncthreads();
  for (int j = 0; j < nkv; ++j) {
    const int buf = j & 1;
    const int64_t key0 = (int64_t)j * BKV;
    if (j + 1 < nkv) load_kv(st, kbase, sh.ks_s, vbase, sh.vs_s, key0 + BKV, S);
    const char* kl = k_lds[buf];
    const char* vl = v_lds[buf];
    // ---- S^T = K Q^T: s[qt][kt] holds keys 16 kt + 4 (lane/16) + e, query column lane % 16
    f32x4_t s[2][4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) s[qt][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const int row = 16 * kt + fr;
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const int ch = (4 * ds + fq) ^ (row & 7);
        const uint4 kf = *reinterpret_cast<const uint4*>(kl + row * kKRow + ch * 16);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) s[qt][kt] = mfma<DT>(kf, qf[qt][ds], s[qt][kt]);
      }
    }
    // ---- online softmax per query column
    const bool need_mask = key0 + BKV > q0 || key0 + BKV > S;  // this wave's rows start at q0
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int64_t q = q0 + 16 * qt + fr;
      float bm = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = s[qt][kt][e] * sl2;
          if (need_mask) {
            const int64_t key = key0 + 16 * kt + 4 * fq + e;
            if (key > q || key >= S) v = -INFINITY;
          }
          s[qt][kt][e] = v;
          bm = fmaxf(bm, v);
        }
      bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
      const float mn = fmaxf(m[qt], bm);
      const float alpha = exp2f(m[qt] - mn);  // m = -inf on the first block: alpha = 0
      float rs = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = exp2f(s[qt][kt][e] - mn);
          s[qt][kt][e] = p;
          rs += p;
        }
      rs += __shfl_xor(rs, 16, 64);
      rs += __shfl_xor(rs, 32, 64);
      l[qt] = l[qt] * alpha + rs;
      m[qt] = mn;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[qt][dt] *= alpha;
    }
    // ---- O^T += V^T P^T over two 32-key steps; P^T tiles (2 ks, 2 ks + 1) form the B operand
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint4 pf[2];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const f32x4_t& a = s[qt][2 * ks];
        const f32x4_t& c = s[qt][2 * ks + 1];
        pf[qt] = make_uint4(pack2<DT>(a[0], a[1]), pack2<DT>(a[2], a[3]), pack2<DT>(c[0], c[1]),
                            pack2<DT>(c[2], c[3]));
      }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const int d = 16 * dt + fr;
        const int u0 = (8 * ks + fq) ^ (d & 15);       // keys 32 ks + 4 (lane/16) .. +3
        const int u1 = (8 * ks + 4 + fq) ^ (d & 15);   // keys 32 ks + 16 + 4 (lane/16) .. +3
        const uint2 v0 = *reinterpret_cast<const uint2*>(vl + d * kVRow + u0 * 8);
        const uint2 v1 = *reinterpret_cast<const uint2*>(vl + d * kVRow + u1 * 8);
        const uint4 vf = make_uint4(v0.x, v0.y, v1.x, v1.y);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) o[qt][dt] = mfma<DT>(vf, pf[qt], o[qt][dt]);
      }
    }
    if (j + 1 < nkv) {
      store_kv(st, k_lds[buf ^ 1], v_lds[buf ^ 1]);
    }
    __syncthreads();
  }

  // ---- O = O^T / l, lse = (m + log2 l) ln 2 (natural log of sum exp(scale * s))
  uint16_t* obase = O + b * sh.os_b + hq * sh.os_h;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t q = q0 + 16 * qt + fr;
    if (q >= S) continue;
    const float inv = 1.0f / l[qt];
    uint16_t* orow = obase + q * sh.os_s;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f32x4_t v = o[qt][dt] * inv;
      *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * fq) =
          make_uint2(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]));
    }
    if (fq == 0 && lse) lse[bh * S + q] = (m[qt] + log2f(l[qt])) * kLn2;
  }
}

// =========================================================================================
// Backward (FlashAttention-2 split): Delta = rowsum(dO * O); dK, dV per key block looping over
// the query heads of its group and the query blocks at or below the diagonal; dQ per query
// block looping over key blocks. P is recomputed from Q, K and the forward's log-sum-exp.
// All products use v_mfma_f32_16x16x32 with the register tile of one product feeding the
// next as an operand: a C tile pair stacked along its rows is an operand whose contraction
// index is that row index (the positions inside a 32-step form a permutation, applied to
// both operands). Transposed copies (Q^T, dO^T, K^T) are written to LDS through an
// in-register 8 x 8 transpose; LDS rows are swizzled (16-B chunks by row & 7 for 256-B rows,
// 8-B units by row & 15 for 128-B rows) so fragment reads are conflict-free.

constexpr int BB = 64;  // rows per staged block in the backward kernels

struct BwdShape {
  int64_t B, HQ, HK, S;
  int64_t qs_b, qs_h, qs_s, ks_b, ks_h, ks_s, vs_b, vs_h, vs_s;
  int64_t os_b, os_h, os_s;   // o and do (same layout)
  int64_t dq_b, dq_h, dq_s;   // dq
  int64_t dk_b, dk_h, dk_s;   // dk and dv (same layout)
  float scale;
};

// Delta[bh, s] = sum_d dO[s, d] * O[s, d]: 16 lanes per row, 8 d each.
template <int DT>
__global__ __launch_bounds__(256) void attn_bwd_delta(const uint16_t* __restrict__ O,
                                                       const uint16_t* __restrict__ dO,
                                                       float* __restrict__ delta, BwdShape sh) {
  const int64_t r = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;  // (b, hq, s) row id
  const int part = threadIdx.x & 15;
  const int64_t total = sh.B * sh.HQ * sh.S;
  const int64_t rc = r < total ? r : total - 1;
  const int64_t bh = rc / sh.S, srow = rc - bh * sh.S;
  const int64_t b = bh / sh.HQ, h = bh - b * sh.HQ;
  const int64_t off = b * sh.os_b + h * sh.os_h + srow * sh.os_s + 8 * part;
  float o8[8], d8[8];
  Vec8<DT>::load(O + off, o8);
  Vec8<DT>::load(dO + off, d8);
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) acc += o8[j] * d8[j];
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (part == 0 && r < total) delta[r] = acc;
}

// Stage an 8 (rows) x 8 (d) block of a [rows, 128] matrix: row-major into a 256-B-row LDS
// tile and transposed into a 128-B-row ([d][row]) LDS tile.
QL_DEV void put_rowmajor(char* __restrict__ lds, const uint4 (&r)[8], int row0, int d0) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = row0 + i;
    const int phys = (d0 >> 3) ^ (row & 7);
    *reinterpret_cast<uint4*>(lds + row * kKRow + phys * 16) = r[i];
  }
}

QL_DEV void put_transposed(char* __restrict__ lds, const uint4 (&r)[8], int row0, int d0) {
  uint4 tr[8];
  transpose8x8(r, tr);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int d = d0 + j;
    const int u0 = (row0 >> 2) ^ (d & 15), u1 = ((row0 >> 2) + 1) ^ (d & 15);
    *reinterpret_cast<uint2*>(lds + d * kVRow + u0 * 8) = make_uint2(tr[j].x, tr[j].y);
    *reinterpret_cast<uint2*>(lds + d * kVRow + u1 * 8) = make_uint2(tr[j].z, tr[j].w);
  }
}

// A fragment of a row-major [rows][128] LDS tile: row, d = 32 ds + 8 (lane/16) .. +7.
QL_DEV uint4 frag_rm(const char* __restrict__ lds, int row, int ds, int fq) {
  const int ch = (4 * ds + fq) ^ (row & 7);
  return *reinterpret_cast<const uint4*>(lds + row * kKRow + ch * 16);
}

// A fragment of a transposed [128][64] LDS tile at row d over the permuted 32-step whose
// positions 0-3 are columns 32 ks + 4 (lane/16) .. +3 and 4-7 are 32 ks + 16 + 4 (lane/16) ..
QL_DEV uint4 frag_tr(const char* __restrict__ lds, int d, int ks, int fq) {
  const int u0 = (8 * ks + fq) ^ (d & 15), u1 = (8 * ks + 4 + fq) ^ (d & 15);
  const uint2 a = *reinterpret_cast<const uint2*>(lds + d * kVRow + u0 * 8);
  const uint2 b = *reinterpret_cast<const uint2*>(lds + d * kVRow + u1 * 8);
  return make_uint4(a.x, a.y, b.x, b.y);
}

// Pack two stacked C tiles (rows 0-15 and 16-31 of a 32-step) into one operand.
template <int DT> QL_DEV uint4 pack_pair(const f32x4_t& a, const f32x4_t& c) {
  return make_uint4(pack2<DT>(a[0], a[1]), pack2<DT>(a[2], a[3]), pack2<DT>(c[0], c[1]),
                    pack2<DT>(c[2], c[3]));
}

// ---- dK, dV: one workgroup per (b, hk, 64-key block). Wave w: query half qh = w & 1 (rows
// 32 qh .. +31 of each 64-row query block), key half kh = w >> 1 (keys 32 kh .. +31). Each
// wave accumulates dV^T and dK^T for its 32 keys over its query rows; the two query halves
// are summed through LDS at the end.
template <int DT>
__global__ __launch_bounds__(256) void attn_bwd_dkdv(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ delta,
    uint16_t* __restrict__ dK, uint16_t* __restrict__ dV, BwdShape sh, int n_kblocks) {
  // per buffer: Q [64][128], Q^T [128][64], dO [64][128], dO^T [128][64], lse2 [64], delta [64]
  constexpr int kTile = BB * kKRow;  // 16 KiB
  constexpr int kBuf = 4 * kTile + 2 * BB * 4;
  __shared__ __attribute__((aligned(16))) char smem[2 * kBuf];
  const int kb = (int)(blockIdx.x % n_kblocks);
  const int64_t bhk = blockIdx.x / n_kblocks;
  const int64_t b = bhk / sh.HK, hk = bhk % sh.HK;
  const int64_t S = sh.S;
  const int group = (int)(sh.HQ / sh.HK);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int fr = lane & 15, fq = lane >> 4;
  const int qh = wave & 1, kh = wave >> 1;
  const int64_t key0 = (int64_t)kb * BB + 32 * kh;  // this wave's first key
  const float sl2 = sh.scale * kLog2e;

  // K and V fragments of this wave's 32 keys (B operands: column key, k = d)
  uint4 kf[2][4], vf[2][4];
  const uint16_t* kbase = K + b * sh.ks_b + hk * sh.ks_h;
  const uint16_t* vbase = V + b * sh.vs_b + hk * sh.vs_h;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int64_t key = key0 + 16 * kt + fr;
    const int64_t kc = key < S ? key : S - 1;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      kf[kt][ds] = *reinterpret_cast<const uint4*>(kbase + kc * sh.ks_s + 32 * ds + 8 * fq);
      vf[kt][ds] = *reinterpret_cast<const uint4*>(vbase + kc * sh.vs_s + 32 * ds + 8 * fq);
    }
  }
  f32x4_t dvt[2][8], dkt[2][8];  // [kt][dt]: rows d = 16 dt + 4 (lane/16) + e, column key
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) dvt[kt][dt] = dkt[kt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int n_qb = (int)((S + BB - 1) / BB);
  const int n_iter = group * (n_qb - kb);  // (head, query block) pairs at or below the diagonal
  // staging: threads 0..127 take an 8 x 8 block of Q, 128..255 of dO; row group (t%128)/16,
  // d group t%16; threads 0..63 also stage lse, 64..127 delta
  const int t = threadIdx.x;
  const int u = t & 127;
  const int srow0 = 8 * (u >> 4), sd0 = 8 * (u & 15);
  uint4 st[8];
  float st_x = 0.f;
  auto load_stage = [&](int it) {
    const int64_t hq = hk * group + it / (n_qb - kb);
    const int qb = kb + it % (n_qb - kb);
    const uint16_t* base = t < 128 ? Q + b * sh.qs_b + hq * sh.qs_h : dO + b * sh.os_b + hq * sh.os_h;
    const int64_t rs = t < 128 ? sh.qs_s : sh.os_s;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t q = (int64_t)qb * BB + srow0 + i;
      const int64_t qc = q < S ? q : S - 1;
      st[i] = *reinterpret_cast<const uint4*>(base + qc * rs + sd0);
    }
    if (t < 128) {
      const int64_t q = (int64_t)qb * BB + (t & 63);
      const int64_t qc = q < S ? q : S - 1;
      const int64_t row = (b * sh.HQ + hq) * S + qc;
      st_x = t < 64 ? lse[row] * kLog2e : delta[row];
    }
  };
  auto store_stage = [&](char* buf) {
    char* rm = buf + (t < 128 ? 0 : 2 * kTile);
    char* tr = buf + (t < 128 ? kTile : 3 * kTile);
    put_rowmajor(rm, st, srow0, sd0);
    put_transposed(tr, st, srow0, sd0);
    if (t < 128) reinterpret_cast<float*>(buf + 4 * kTile)[t] = st_x;  // lse2 [64], delta [64]
  };

  if (n_iter > 0) {
    load_stage(0);
    store_stage(smem);
  }
  __syncthreads();
  for (int it = 0; it < n_iter; ++it) {
    char* buf = smem + (it & 1) * kBuf;
    if (it + 1 < n_iter) load_stage(it + 1);
    const int qb = kb + it % (n_qb - kb);
    const int64_t qrow0 = (int64_t)qb * BB + 32 * qh;  // this wave's first query row
    const char* q_rm = buf;
    const char* q_tr = buf + kTile;
    const char* do_rm = buf + 2 * kTile;
    const char* do_tr = buf + 3 * kTile;
    const float* lse2 = reinterpret_cast<const float*>(buf + 4 * kTile);
    const float* dlt = lse2 + BB;
    // S and dP tiles [qt][kt]: rows q = 32 qh + 16 qt + 4 (lane/16) + e, column key 16 kt + lane%16
    f32x4_t sp[2][2], dp[2][2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) sp[qt][kt] = dp[qt][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const int row = 32 * qh + 16 * qt + fr;
        const uint4 qa = frag_rm(q_rm, row, ds, fq);
        const uint4 da = frag_rm(do_rm, row, ds, fq);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          sp[qt][kt] = mfma<DT>(qa, kf[kt][ds], sp[qt][kt]);
          dp[qt][kt] = mfma<DT>(da, vf[kt][ds], dp[qt][kt]);
        }
      }
    }
    // P = exp2(S log2e scale - lse2), dS = P (dP - delta); causal / length mask -> 0
    const bool diag = qb == kb;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 32 * qh + 16 * qt + 4 * fq + e;
        const int64_t q = (int64_t)qb * BB + r;
        const float l2 = lse2[r], dl = dlt[r];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          const int64_t key = key0 + 16 * kt + fr;
          float p = exp2f(sp[qt][kt][e] * sl2 - l2);
          if ((diag && key > q) || q >= S) p = 0.f;
          sp[qt][kt][e] = p;
          dp[qt][kt][e] = p * (dp[qt][kt][e] - dl);
        }
      }
    // dV^T += dO^T P ; dK^T += Q^T dS   (contraction over this wave's 32 query rows)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const uint4 pb = pack_pair<DT>(sp[0][kt], sp[1][kt]);
      const uint4 sb = pack_pair<DT>(dp[0][kt], dp[1][kt]);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const int d = 16 * dt + fr;
        dvt[kt][dt] = mfma<DT>(frag_tr(do_tr, d, qh, fq), pb, dvt[kt][dt]);
        dkt[kt][dt] = mfma<DT>(frag_tr(q_tr, d, qh, fq), sb, dkt[kt][dt]);
      }
    }
    if (it + 1 < n_iter) store_stage(smem + ((it + 1) & 1) * kBuf);
    __syncthreads();
  }

  // sum the two query halves (wave pairs with the same kh) through LDS, then store
  float* red = reinterpret_cast<float*>(smem);  // [kh][kt][dt][lane] f32x4 of dV then dK
  auto slot = [&](int which, int kt, int dt) -> f32x4_t* {
    return reinterpret_cast<f32x4_t*>(red) + ((((kh * 2 + which) * 2 + kt) * 8 + dt) * 64 + lane);
  };
  if (qh == 1) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        *slot(0, kt, dt) = dvt[kt][dt];
        *slot(1, kt, dt) = dkt[kt][dt];
      }
  }
  __syncthreads();
  if (qh == 0) {
    uint16_t* dkb = dK + b * sh.dk_b + hk * sh.dk_h;
    uint16_t* dvb = dV + b * sh.dk_b + hk * sh.dk_h;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int64_t key = key0 + 16 * kt + fr;
      if (key >= S) continue;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const f32x4_t v = dvt[kt][dt] + *slot(0, kt, dt);
        const f32x4_t k4 = (dkt[kt][dt] + *slot(1, kt, dt)) * sh.scale;
        const int d = 16 * dt + 4 * fq;
        *reinterpret_cast<uint2*>(dvb + key * sh.dk_s + d) =
            make_uint2(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]));
        *reinterpret_cast<uint2*>(dkb + key * sh.dk_s + d) =
            make_uint2(pack2<DT>(k4[0], k4[1]), pack2<DT>(k4[2], k4[3]));
      }
    }
  }
}

// ---- dQ: one workgroup per (b, hq, 128-row query block); wave w owns rows 32 w .. +31.
template <int DT>
__global__ __launch_bounds__(256) void attn_bwd_dq(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ delta,
    uint16_t* __restrict__ dQ, BwdShape sh, int n_qblocks) {
  // per buffer: K [64][128], K^T [128][64], V [64][128]
  constexpr int kTile = BB * kKRow;
  constexpr int kBuf = 3 * kTile;
  __shared__ __attribute__((aligned(16))) char smem[2 * kBuf];
  const int qb = n_qblocks - 1 - (int)(blockIdx.x % n_qblocks);  // heaviest first
  const int64_t bh = blockIdx.x / n_qblocks;
  const int64_t b = bh / sh.HQ, hq = bh % sh.HQ;
  const int64_t hk = hq / (sh.HQ / sh.HK);
  const int64_t S = sh.S;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int fr = lane & 15, fq = lane >> 4;
  const int64_t q0 = (int64_t)qb * BQ + 32 * wave;
  const float sl2 = sh.scale * kLog2e;

  // Q and dO fragments (B operands: column q = lane%16, k = d); lse2 and delta per column
  uint4 qf[2][4], df[2][4];
  float l2[2], dl[2];
  const uint16_t* qbase = Q + b * sh.qs_b + hq * sh.qs_h;
  const uint16_t* dobase = dO + b * sh.os_b + hq * sh.os_h;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t q = q0 + 16 * qt + fr;
    const int64_t qc = q < S ? q : S - 1;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      qf[qt][ds] = *reinterpret_cast<const uint4*>(qbase + qc * sh.qs_s + 32 * ds + 8 * fq);
      df[qt][ds] = *reinterpret_cast<const uint4*>(dobase + qc * sh.os_s + 32 * ds + 8 * fq);
    }
    l2[qt] = lse[bh * S + qc] * kLog2e;
    dl[qt] = delta[bh * S + qc];
  }
  f32x4_t dqt[2][8];  // [qt][dt]: rows d = 16 dt + 4 (lane/16) + e, column q
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) dqt[qt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int64_t q_end = (int64_t)(qb + 1) * BQ;
  const int64_t kv_end = q_end < S ? q_end : S;
  const int nkv = (int)((kv_end + BB - 1) / BB);
  // staging: threads 0..127 an 8 x 8 block of K (row-major + transposed), 128..255 of V
  const int t = threadIdx.x;
  const int u = t & 127;
  const int srow0 = 8 * (u >> 4), sd0 = 8 * (u & 15);
  const uint16_t* sbase = t < 128 ? K + b * sh.ks_b + hk * sh.ks_h : V + b * sh.vs_b + hk * sh.vs_h;
  const int64_t srs = t < 128 ? sh.ks_s : sh.vs_s;
  uint4 st[8];
  auto load_stage = [&](int j) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t key = (int64_t)j * BB + srow0 + i;
      const int64_t kc = key < S ? key : S - 1;
      st[i] = *reinterpret_cast<const uint4*>(sbase + kc * srs + sd0);
    }
  };
  auto store_stage = [&](char* buf) {
    if (t < 128) {
      put_rowmajor(buf, st, srow0, sd0);
      put_transposed(buf + kTile, st, srow0, sd0);
    } else {
      put_rowmajor(buf + 2 * kTile, st, srow0, sd0);
    }
  };
  load_stage(0);
  store_stage(smem);
  __syncthreads();
  for (int j = 0; j < nkv; ++j) {
    char* buf = smem + (j & 1) * kBuf;
    if (j + 1 < nkv) load_stage(j + 1);
    const char* k_rm = buf;
    const char* k_tr = buf + kTile;
    const char* v_rm = buf + 2 * kTile;
    const int64_t key0 = (int64_t)j * BB;
    // S^T and dP^T tiles [qt][kt]: rows key 16 kt + 4 (lane/16) + e, column q
    f32x4_t sp[2][4], dp[2][4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) sp[qt][kt] = dp[qt][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const int row = 16 * kt + fr;
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const uint4 ka = frag_rm(k_rm, row, ds, fq);
        const uint4 va = frag_rm(v_rm, row, ds, fq);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          sp[qt][kt] = mfma<DT>(ka, qf[qt][ds], sp[qt][kt]);
          dp[qt][kt] = mfma<DT>(va, df[qt][ds], dp[qt][kt]);
        }
      }
    }
    const bool need_mask = key0 + BB > q0 || key0 + BB > S;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int64_t q = q0 + 16 * qt + fr;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float p = exp2f(sp[qt][kt][e] * sl2 - l2[qt]);
          if (need_mask) {
            const int64_t key = key0 + 16 * kt + 4 * fq + e;
            if (key > q || key >= S) p = 0.f;
          }
          dp[qt][kt][e] = p * (dp[qt][kt][e] - dl[qt]);
        }
    }
    // dQ^T += K^T dS^T (contraction over the 64 keys in two permuted 32-steps)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint4 sb[2];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) sb[qt] = pack_pair<DT>(dp[qt][2 * ks], dp[qt][2 * ks + 1]);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint4 ka = frag_tr(k_tr, 16 * dt + fr, ks, fq);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) dqt[qt][dt] = mfma<DT>(ka, sb[qt], dqt[qt][dt]);
      }
    }
    if (j + 1 < nkv) store_stage(smem + ((j + 1) & 1) * kBuf);
    __syncthreads();
  }
  uint16_t* dqb = dQ + b * sh.dq_b + hq * sh.dq_h;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t q = q0 + 16 * qt + fr;
    if (q >= S) continue;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f32x4_t v = dqt[qt][dt] * sh.scale;
      *reinterpret_cast<uint2*>(dqb + q * sh.dq_s + 16 * dt + 4 * fq) =
          make_uint2(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]));
    }
  }
}

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

extern "C" int64_t qlora_attn_bwd_workspace_size(int64_t B, int64_t HQ, int64_t S) {
  if (B <= 0 || HQ <= 0 || S <= 0) return 0;
  return B * HQ * S * (int64_t)sizeof(float);
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
  if (workspace_bytes < qlora_attn_bwd_workspace_size(B, HQ, S) || !workspace ||
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
  float* delta = static_cast<float*>(workspace);
  const int64_t rows = B * HQ * S;
  const int n_kblocks = (int)((S + BB - 1) / BB);
  const int n_qblocks = (int)((S + BQ - 1) / BQ);
  if (B * HK * n_kblocks > INT32_MAX || B * HQ * n_qblocks > INT32_MAX) return QL_EINVAL;
#define QL_ATTN_BWD(DTC)                                                                          \
  do {                                                                                            \
    hipLaunchKernelGGL((attn_bwd_delta<DTC>), dim3((unsigned)((rows * 16 + 255) / 256)), dim3(256), \
                       0, s, (const uint16_t*)o, (const uint16_t*)d_o, delta, sh);                \
    hipLaunchKernelGGL((attn_bwd_dkdv<DTC>), dim3((unsigned)(B * HK * n_kblocks)), dim3(256), 0, s, \
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,                \
                       (const uint16_t*)d_o, lse, delta, (uint16_t*)dk, (uint16_t*)dv, sh,        \
                       n_kblocks);                                                                \
    hipLaunchKernelGGL((attn_bwd_dq<DTC>), dim3((unsigned)(B * HQ * n_qblocks)), dim3(256), 0, s,  \
                       (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,                \
                       (const uint16_t*)d_o, lse, delta, (uint16_t*)dq, sh, n_qblocks);           \
  } while (0)
  if (dtype == QL_BF16) QL_ATTN_BWD(QL_BF16);
  else QL_ATTN_BWD(QL_F16);
#undef QL_ATTN_BWD
  return ql_launch_status();
}
