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
//   - workgroup tile 256 x BN x 64 with BN = 256 or 224, 256 threads = 4 waves, one workgroup
//     per CU. The products are v_mfma_f32_32x32x16: a single wave per SIMD issues them at the
//     full matrix-core rate (one per 32 cycles), where it can only issue the 16x16x32 form
//     about once per 25 cycles instead of 16. Each wave owns BI x BJ blocks of 32 x 32 (16 fp32
//     per lane each, in AGPRs): 256 wide as 2 x 2 waves of 4 x 4 blocks, 224 wide as 4 x 1
//     waves of 2 x 7 blocks;
//   - operands go global -> LDS with global_load_lds_dwordx4 (no VGPR staging, no ds_write):
//     each wave instruction fills 1 KiB of LDS = 8 rows of 64 k. Rows are 128 B with the
//     16-B chunks XOR-swizzled by s(row) = ((row >> 1) & 3) | ((row >> 3) & 1) << 2. The LDS
//     has 64 banks (256 B, two rows), and a ds_read_b128 cycle serves 16 lanes, 8-lane
//     blocks b and b ^ 3 together (lanes 0..7 with 24..31, 8..15 with 16..23; measured with
//     SQ_LDS_BANK_CONFLICT). Fragment reads put lane l on row l % 32, so a cycle meets rows
//     r .. r + 7 and r ^ 24 .. +7: s takes 8 distinct values over the 8 even (and the 8 odd)
//     rows of those, and every read is conflict-free (s = row & 7 cost 4 stall cycles per
//     read);
//   - two LDS stages, software-pipelined across K steps: each step multiplies the first 32-k
//     half of its stage while reading the second half's fragments, meets the other waves at
//     the one barrier of the step, starts the DMA of step k+2 into the stage just consumed
//     (each load placed behind one MFMA, first thing after the barrier, so it has the most
//     time to land) and multiplies the second half while reading the first-half fragments of
//     step k+1. Scheduling barriers keep that instruction order;
//   - workgroup ids are remapped so that the tiles one XCD runs at a time are neighbours
//     (XCDs take workgroups round-robin; each has its own L2), then rastered in groups of 4
//     tile rows so that concurrently running tiles share A and B panels in L2;
//   - a second K segment C += A2 B2^T (K2 % 64 == 0, at most 128 columns, same M and N) can
//     join the first: the rank-16 LoRA term of a LoRA linear rides along as one extra K step
//     of the base GEMM (x W^T + u (sB)^T with u, sB zero-padded to 64 columns) instead of
//     separate skinny GEMMs and an elementwise add. Its steps come first, loaded by the
//     prologue, so every load inside the K loop is a step of the first segment; for operands
//     with a multiple of 8 rows those loads use addresses built once per tile (Panel), and a
//     step only adds its k offset;
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
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

constexpr int BM = 256, BK = 64;
constexpr int kThreads = 256;
constexpr int kRowBytes = BK * 2;              // 128 B: one tile row of 64 k
constexpr int kATileBytes = BM * kRowBytes;    // 32 KiB: the A operand, one stage
constexpr int kGroupM = 4;
constexpr int kPrologueSteps = 2;              // the second K segment fits in the prologue

// Tile width NB x 32 and the wave layout of a 256 x BN tile: WM x WN waves, each owning
// BI x BJ blocks of 32 x 32.
template <int NB> struct Layout;
template <> struct Layout<8> { static constexpr int WM = 2, WN = 2, BI = 4, BJ = 4; };
template <> struct Layout<7> { static constexpr int WM = 4, WN = 1, BI = 2, BJ = 7; };
template <int NB> constexpr int bn_of() { return 32 * NB; }
// one stage: A (256 rows) then B (BN rows): 64 KiB at BN = 256
template <int NB> constexpr int stage_bytes() { return kATileBytes + bn_of<NB>() * kRowBytes; }

// D[32 x 32] += a[32 x 16] b[16 x 32]: lane l supplies row l%32, k 8(l/32) .. +7 of each
// operand and holds D[8i + 4(l/32) + j][l%32] in element 4i + j.
template <int DT> QL_DEV f32x16_t mfma(const uint4& a, const uint4& b, f32x16_t c);
template <> QL_DEV f32x16_t mfma<QL_BF16>(const uint4& a, const uint4& b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <> QL_DEV f32x16_t mfma<QL_F16>(const uint4& a, const uint4& b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Issue this wave's share of one operand tile (32 R8 rows x 64 k starting at (row0, k0)) as
// R8 direct-to-LDS loads. Instruction j of wave w fills tile rows r0 = (4j + w) * 8 .. +7;
// lane l writes LDS bytes [16 l, 16 l + 16) of that 1 KiB span, i.e. row r0 + l/8,
// physical chunk l%8, which holds logical chunk (l%8) ^ s(row) of the row. Bit 3 of that row
// is w & 1 for every j, so s(row) = ((l/8 >> 1) & 3) | (w & 1) << 2 is fixed per lane.
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
  t.chunk16 = (uint32_t)(((lane & 7) ^ (((t.rsub >> 1) & 3) | (t.wave & 1) << 2)) * 16);
  return t;
}

template <int R8 = 8>  // tile rows / 32: 7 or 8 (224 or 256 rows)
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

// load_tile with each load written as inline assembly, for the prologue. The compiler's
// wait-count pass sees the builtin direct-to-LDS loads of one LDS array as possibly
// overlapping, and waited for all of them (vmcnt(0)) between the A and B loads of each stage
// and before the first fragment reads: four HBM round trips in a row before the first
// product. Hidden from it, both stages' loads go out together, and the kernel's own
// s_waitcnt vmcnt + barrier are the only waits. (s_nop 4: the wait states a write of M0
// needs before a vector memory instruction reads it; inline assembly gets no hazard padding.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is clobbered on purpose
QL_DEV void dma_hidden(const char* sbase, uint32_t voff, char* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr_t)lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(m0)
               : "memory", "m0");
}
#pragma clang diagnostic pop

template <int R8 = 8>
QL_DEV void load_tile_hidden(const TileLoader& t, const uint16_t* __restrict__ X, int64_t ld,
                             int64_t row0, int64_t rows, int64_t k0, char* __restrict__ lds_tile) {
#pragma unroll
  for (int j = 0; j < R8; ++j) {
    const int r0 = (4 * j + t.wave) * 8;
    const int64_t grow0 = row0 + r0;
    const int64_t base_row = grow0 < rows ? grow0 : rows - 1;
    const int64_t r = (grow0 + t.rsub) < rows ? grow0 + t.rsub : rows - 1;
    const uint32_t off = (uint32_t)(r - base_row) * (uint32_t)(ld * 2) + t.chunk16;
    dma_hidden(reinterpret_cast<const char*>(X + base_row * ld + k0), off,
               lds_tile + r0 * kRowBytes);
  }
}

// Prologue step t (second-segment steps first) of a dense tile: 8 + NB hidden loads per wave.
// A plain function with its operands by value (a capturing lambda left them in memory, and
// the reloads' waits drained the loads in flight).
template <int NB>
QL_DEV void prologue_dense(const TileLoader& la, const uint16_t* A, int64_t lda,
                           const uint16_t* B, int64_t ldb, const uint16_t* A2, int64_t lda2,
                           const uint16_t* B2, int64_t ldb2, int nk2, int64_t kb, int64_t m0,
                           int64_t n0, int64_t M, int64_t N, int t, char* stage) {
  const bool s2 = t < nk2;
  const int64_t k0 = s2 ? (int64_t)t * BK : kb + (int64_t)(t - nk2) * BK;
  load_tile_hidden(la, s2 ? A2 : A, s2 ? lda2 : lda, m0, M, k0, stage);
  load_tile_hidden<NB>(la, s2 ? B2 : B, s2 ? ldb2 : ldb, n0, N, k0, stage + kATileBytes);
}

// The same loads for an operand whose row count is a multiple of 8, with the addresses
// computed once per tile: every 8-row group a load covers is then either wholly inside the
// operand or wholly past its end (a group past the end re-reads the last 8 rows, tile rows
// that are never stored), so each load keeps a wave-uniform row base and all of them share
// one lane offset; a K step only adds its k offset.
template <int R8>
struct Panel {
  const char* base[R8];  // wave-uniform: first row of load j at the panel's first k
  uint32_t off;          // lane offset: (lane / 8) rows + physical 16-B chunk
};

template <int R8>
QL_DEV void panel_init(Panel<R8>& p, const TileLoader& t, const uint16_t* __restrict__ X,
                       int64_t ld, int64_t row0, int64_t rows, int64_t k0) {
#pragma unroll
  for (int j = 0; j < R8; ++j) {
    const int64_t g = row0 + (4 * j + t.wave) * 8;
    p.base[j] = reinterpret_cast<const char*>(X + (g < rows ? g : rows - 8) * ld + k0);
  }
  p.off = (uint32_t)(t.rsub * ld * 2) + t.chunk16;
}

template <int R8>
QL_DEV void panel_issue(const Panel<R8>& p, const TileLoader& t, uint32_t kbytes,
                        char* __restrict__ lds_tile) {
  const uint32_t off = p.off + kbytes;
#pragma unroll
  for (int j = 0; j < R8; ++j)
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)(p.base[j] + off),
                                     (lds_ptr_t)(lds_tile + (4 * j + t.wave) * 8 * kRowBytes), 16,
                                     0, 0);
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

template <int NB>
struct Frags {
  uint4 a[2][Layout<NB>::BI];  // [16-k block][row block]
  uint4 b[2][Layout<NB>::BJ];  // [16-k block][column block]
};

// Fragment reads of one 32-k half of a stage: lane l reads row l%32 of each block, logical
// chunk 4 half + 2 kk + l/32 for the half's 16-k blocks kk = 0, 1.
template <int NB>
QL_DEV void read_frags(const char* __restrict__ stage, int half, int wm, int wn, int lane,
                       Frags<NB>& f) {
  using L = Layout<NB>;
  const int r = lane & 31;
  const char* as = stage + (wm * L::BI * 32 + r) * kRowBytes;
  const char* bs = stage + kATileBytes + (wn * L::BJ * 32 + r) * kRowBytes;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const int c = ((half * 4 + kk * 2 + (lane >> 5)) ^ (((r >> 1) & 3) | ((r >> 3) & 1) << 2)) * 16;
#pragma unroll
    for (int i = 0; i < L::BI; ++i) f.a[kk][i] = *reinterpret_cast<const uint4*>(as + i * 32 * kRowBytes + c);
#pragma unroll
    for (int j = 0; j < L::BJ; ++j) f.b[kk][j] = *reinterpret_cast<const uint4*>(bs + j * 32 * kRowBytes + c);
  }
}

// B fragments go in as the first operand, so each lane's accumulator holds 4 consecutive
// output columns of one output row (element 4g + e: row l%32, column 8g + 4(l/32) + e).
template <int IT, int NB>
QL_DEV void mma_half(f32x16_t (&acc)[Layout<NB>::BI][Layout<NB>::BJ], const Frags<NB>& f) {
  using L = Layout<NB>;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int i = 0; i < L::BI; ++i)
#pragma unroll
      for (int j = 0; j < L::BJ; ++j) acc[i][j] = mfma<IT>(f.b[kk][j], f.a[kk][i], acc[i][j]);
}

// One K step, software-pipelined across steps. On entry f0 holds the first-half fragments of
// stage `cur` (read during the previous step) and the DMA of the next step into `nxt` is in
// flight. The step reads the second half of `cur` while multiplying the first; then every
// wave waits for its DMA of the next step and meets at the barrier (after it, all of `cur`
// has been read by every wave), starts the DMA of the step after next into `cur` through
// `issue` (each load placed behind one MFMA, first thing after the barrier, so it has the
// most time to land), and reads the first half of `nxt` while multiplying the second half of
// `cur`. `cur` and `nxt` are restrict-qualified so the compiler's wait-count pass does not
// make these reads wait for the DMA into `cur`. Per half step: RH fragment reads and MF
// MFMAs; the second half also issues the G DMA loads.
template <int IT, int NB, typename Issue>
QL_DEV void mma_step_pipe(f32x16_t (&acc)[Layout<NB>::BI][Layout<NB>::BJ], Frags<NB>& f0,
                          char* __restrict__ cur, char* __restrict__ nxt, const Issue& issue,
                          int wm, int wn, int lane) {
  using L = Layout<NB>;
  constexpr int RH = 2 * (L::BI + L::BJ), MF = 2 * L::BI * L::BJ, G = 8 + NB;
  constexpr int REST = MF - G;                    // second-half MFMAs left for the reads
  constexpr int DBL = RH > REST ? RH - REST : 0;  // of which carry two reads
  static_assert(MF - 1 - RH >= 0 && REST >= DBL, "schedule does not fit the tile");
  Frags<NB> f1;
  read_frags<NB>(cur, 1, wm, wn, lane, f1);
  mma_half<IT, NB>(acc, f0);
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
  for (int t = 0; t < RH; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, MF - 1 - RH, 0);
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  issue(cur);
  read_frags<NB>(nxt, 0, wm, wn, lane, f0);
  mma_half<IT, NB>(acc, f1);
#pragma unroll
  for (int t = 0; t < G; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
  }
#pragma unroll
  for (int t = 0; t < DBL; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
  }
#pragma unroll
  for (int t = 0; t < RH - 2 * DBL; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
  }
  if constexpr (REST - DBL - (RH - 2 * DBL) > 0)
    __builtin_amdgcn_sched_group_barrier(0x008, REST - DBL - (RH - 2 * DBL), 1);
}

// ---- B as packed NF4 (dequantised on the way into LDS) ----------------------------------------
// The B operand can be an NF4 weight W [N, K] (packed two per byte, high nibble first; one
// absmax per block of bs = 2^log2_bs >= 64 consecutive weights of a row, bs dividing K) instead
// of a 16-bit matrix. Thread t of the workgroup owns B tile row t: per K step it loads the
// row's 32 packed bytes and its block scale one step ahead into registers, and after the step's
// barrier dequantises the 64 weights into that row of the LDS stage, in the swizzled layout the
// fragment reads expect, with the dequant kernel's operation order (scale = code2[q] * absmax2,
// then + offset, two fp32 roundings; product nf4[c] * scale rounded to fp32, then to bf16/fp16
// by RNE): the products see exactly the 16-bit W that qlora_nf4_dequant writes.
// The 16 products of a block are built once, then each weight is a table lookup: the table's
// low and high bytes sit in two 16-byte planes, and v_perm_b32 selects 4 entries at a time.
enum { kBDense = 0, kBNf4Nested = 1, kBNf4Plain = 2 };

struct Nf4Operand {
  const uint8_t* packed;  // weight (n, k) in byte (n K + k) / 2
  const void* absmax;     // uint8 codes (nested) or fp32 absmax, one per block
  const float* absmax2;   // nested: second-level scale per 2^log2_bs2 blocks
  const float* code2;     // nested: 256-entry code table
  const float* nf4;       // the 16 NF4 levels
  float offset;
  int log2_bs, log2_bs2;
};

// In-flight state of one thread's B row for the next K step.
struct Nf4Row {
  const uint8_t* row;  // packed bytes of (clamped) row n, k = 0
  int64_t w0;          // weight index of (n, 0)
  uint4 pk[2];         // 64 weights, k0 .. k0 + 63
  uint32_t code;       // absmax code (nested) or the fp32 absmax bits
  float a2;            // second-level scale (nested)
};

template <int BQ>
QL_DEV void nf4_issue(Nf4Row& r, const Nf4Operand& op, int64_t k0) {
  const uint4* p = reinterpret_cast<const uint4*>(r.row + (k0 >> 1));
  r.pk[0] = p[0];
  r.pk[1] = p[1];
  const int64_t blk = (r.w0 + k0) >> op.log2_bs;
  if constexpr (BQ == kBNf4Nested) {
    r.code = static_cast<const uint8_t*>(op.absmax)[blk];
    r.a2 = op.absmax2[blk >> op.log2_bs2];
  } else {
    r.code = __float_as_uint(static_cast<const float*>(op.absmax)[blk]);
    r.a2 = 0.f;
  }
}

// The product must reach fp32 before the 16-bit conversion (the backend would otherwise fuse
// multiply and conversion into one v_fma_mix with a single rounding).
QL_DEV float nf4_round32(float x) {
  asm("" : "+v"(x));
  return x;
}

template <int IT>
QL_DEV uint32_t nf4_pack2(float lo, float hi) {
  if constexpr (IT == QL_BF16) return pack_bf16x2(lo, hi);
  else return pack_f16x2(lo, hi);
}

// Byte j of the result: table entry idx.byte[j] (each 0..15) of the planes (lo and hi bytes of
// the 16 entries, four per dword), low or high byte.
QL_DEV uint32_t nf4_plane_lookup(const uint32_t (&pl)[4], uint32_t sel7, uint32_t pick) {
  const uint32_t a = __builtin_amdgcn_perm(pl[1], pl[0], sel7);  // entries 0..7
  const uint32_t b = __builtin_amdgcn_perm(pl[3], pl[2], sel7);  // entries 8..15
  return __builtin_amdgcn_perm(b, a, pick);
}

// A block's 16 products as byte planes, and the packed words of its last 4 chunks: what the
// second half of a row's dequantisation needs, carried from one K step to the next.
struct Nf4Pending {
  uint32_t lo[4], hi[4];
  uint32_t d[4];
};

// Block scale and table planes of row state r (the dequant kernel's fp32 order).
template <int BQ, int IT>
QL_DEV void nf4_planes(const Nf4Row& r, const Nf4Operand& op, const float (&nf4)[16],
                       const float* code2_lds, uint32_t (&lo)[4], uint32_t (&hi)[4]) {
#pragma clang fp contract(off)
  float s;
  if constexpr (BQ == kBNf4Nested) {
    s = code2_lds[r.code] * r.a2;
    s = s + op.offset;
  } else {
    s = __uint_as_float(r.code);
  }
  uint32_t pair[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    pair[i] = nf4_pack2<IT>(nf4_round32(nf4[2 * i] * s), nf4_round32(nf4[2 * i + 1] * s));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    lo[j] = __builtin_amdgcn_perm(pair[2 * j + 1], pair[2 * j], 0x06040200u);
    hi[j] = __builtin_amdgcn_perm(pair[2 * j + 1], pair[2 * j], 0x07050301u);
  }
}

// Half h of an NF4 chunk: weights 4h .. 4h + 3 of the 8 in packed word d (byte i holds weight
// 2i in its high nibble, 2i + 1 in its low one), as two dwords of 16-bit pairs.
QL_DEV void nf4_half(const uint32_t (&lo)[4], const uint32_t (&hi)[4], uint32_t d, int h,
                     uint32_t& w0, uint32_t& w1) {
  const uint32_t even = (d >> 4) & 0x0f0f0f0fu, odd = d & 0x0f0f0f0fu;
  const uint32_t idx = __builtin_amdgcn_perm(even, odd, h ? 0x03070206u : 0x01050004u);
  const uint32_t sel7 = idx & 0x07070707u;
  const uint32_t pick = ((idx >> 1) & 0x04040404u) | 0x03020100u;
  const uint32_t l = nf4_plane_lookup(lo, sel7, pick);
  const uint32_t u = nf4_plane_lookup(hi, sel7, pick);
  w0 = __builtin_amdgcn_perm(u, l, 0x05010400u);
  w1 = __builtin_amdgcn_perm(u, l, 0x07030602u);
}

// Chunks c0 .. c0 + 3 of a row (packed words d[0..3], 8 weights each) into its LDS row
// (128 B, 16-B chunks swizzled by swz).
QL_DEV void nf4_chunks(const uint32_t (&lo)[4], const uint32_t (&hi)[4], const uint32_t* d,
                       int c0, char* __restrict__ lds_row, uint32_t swz) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint32_t w[4];
    nf4_half(lo, hi, d[c], 0, w[0], w[1]);
    nf4_half(lo, hi, d[c], 1, w[2], w[3]);
    *reinterpret_cast<uint4*>(lds_row + 16 * ((c0 + c) ^ swz)) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Dequantise a whole row (the prologue's steps): planes, then all 8 chunks; when `pend` is
// given, only chunks 0..3 are stored and the rest is left in it for the first K step.
template <int BQ, int IT>
QL_DEV void nf4_store_row(const Nf4Row& r, const Nf4Operand& op, const float (&nf4)[16],
                          const float* code2_lds, char* __restrict__ lds_row, uint32_t swz,
                          Nf4Pending* pend) {
  uint32_t lo[4], hi[4];
  nf4_planes<BQ, IT>(r, op, nf4, code2_lds, lo, hi);
  const uint32_t d0[4] = {r.pk[0].x, r.pk[0].y, r.pk[0].z, r.pk[0].w};
  const uint32_t d1[4] = {r.pk[1].x, r.pk[1].y, r.pk[1].z, r.pk[1].w};
  nf4_chunks(lo, hi, d0, 0, lds_row, swz);
  if (pend) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pend->lo[j] = lo[j];
      pend->hi[j] = hi[j];
      pend->d[j] = d1[j];
    }
  } else {
    nf4_chunks(lo, hi, d1, 4, lds_row, swz);
  }
}

// MFMAs 4s .. 4s + 3 of a half step (16-k block s / 4, row block s % 4, all 4 column blocks).
template <int IT>
QL_DEV void mma_slice(f32x16_t (&acc)[4][4], const Frags<8>& f, int s) {
  const int kk = s >> 2, i = s & 3;
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[i][j] = mfma<IT>(f.b[kk][j], f.a[kk][i], acc[i][j]);
}

// Part p (0..3) of read_frags: the A (p even) or B (p odd) fragments of 16-k block p / 2.
QL_DEV void read_frags_part(const char* __restrict__ stage, int half, int wm, int wn, int lane,
                            Frags<8>& f, int p) {
  const int r = lane & 31;
  const int kk = p >> 1;
  const int c = ((half * 4 + kk * 2 + (lane >> 5)) ^ (((r >> 1) & 3) | ((r >> 3) & 1) << 2)) * 16;
  if (p & 1) {
    const char* bs = stage + kATileBytes + (wn * 4 * 32 + r) * kRowBytes;
#pragma unroll
    for (int j = 0; j < 4; ++j) f.b[kk][j] = *reinterpret_cast<const uint4*>(bs + j * 32 * kRowBytes + c);
  } else {
    const char* as = stage + (wm * 4 * 32 + r) * kRowBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) f.a[kk][i] = *reinterpret_cast<const uint4*>(as + i * 32 * kRowBytes + c);
  }
}

// One K step of the NF4-B kernel: mma_step_pipe's products, fragment reads and barrier, with
// B dequantised by the threads, cut into 8 slices of 4 MFMAs per half (scheduling fences
// between slices keep the dequantisation's VALU work spread between the products):
//   first half:  chunks 4..7 of step kt + 1's row (planes and words carried in `pend`), half a
//                chunk per slice, into `nxt` (no wave reads it before this step's barrier);
//   second half: A's DMA of step kt + 2 into `cur` (issue_a), the packed bytes and scale of
//                step kt + 3 into `brow` (issue_b), then step kt + 2's row (landed at this
//                step's barrier): planes, chunks 0..3 into `cur`, chunks 4..7 into `pend`;
//                the first-half fragments of `nxt` are read a quarter per slice.
template <int BQ, int IT, typename IssueA, typename IssueB>
QL_DEV void mma_step_pipe_nf4(f32x16_t (&acc)[4][4], Frags<8>& f0, char* __restrict__ cur,
                              char* __restrict__ nxt, const IssueA& issue_a, const IssueB& issue_b,
                              Nf4Row& brow, Nf4Pending& pend, const Nf4Operand& op,
                              const float (&nf4)[16], const float* code2_lds, int row_off,
                              uint32_t swz, int wm, int wn, int lane) {
  Frags<8> f1;
  read_frags<8>(cur, 1, wm, wn, lane, f1);
  uint32_t w[4];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int c = s >> 1, h = s & 1;
    nf4_half(pend.lo, pend.hi, pend.d[c], h, w[2 * h], w[2 * h + 1]);
    if (h)
      *reinterpret_cast<uint4*>(nxt + row_off + 16 * ((4 + c) ^ swz)) =
          make_uint4(w[0], w[1], w[2], w[3]);
    mma_slice<IT>(acc, f0, s);
    __builtin_amdgcn_sched_barrier(0);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  // slice 0: A's DMA, the next row's loads
  issue_a(cur);
  const Nf4Row now = brow;
  issue_b(brow);
  mma_slice<IT>(acc, f1, 0);
  __builtin_amdgcn_sched_barrier(0);
  // slices 1, 2: this row's scale and table planes
  uint32_t lo[4], hi[4];
  nf4_planes<BQ, IT>(now, op, nf4, code2_lds, lo, hi);
  read_frags_part(nxt, 0, wm, wn, lane, f0, 0);
  mma_slice<IT>(acc, f1, 1);
  __builtin_amdgcn_sched_barrier(0);
  read_frags_part(nxt, 0, wm, wn, lane, f0, 1);
  mma_slice<IT>(acc, f1, 2);
  __builtin_amdgcn_sched_barrier(0);
  // slices 3..7: the 8 half-chunks of chunks 0..3, [first[s], first[s + 1]) in slice s
  const uint32_t d0[4] = {now.pk[0].x, now.pk[0].y, now.pk[0].z, now.pk[0].w};
  constexpr int first[9] = {0, 0, 0, 0, 1, 3, 5, 7, 8};
#pragma unroll
  for (int s = 3; s < 8; ++s) {
#pragma unroll
    for (int e = first[s]; e < first[s + 1]; ++e) {
      const int c = e >> 1, h = e & 1;
      nf4_half(lo, hi, d0[c], h, w[2 * h], w[2 * h + 1]);
      if (h)
        *reinterpret_cast<uint4*>(cur + row_off + 16 * (c ^ swz)) =
            make_uint4(w[0], w[1], w[2], w[3]);
    }
    if (s == 3) read_frags_part(nxt, 0, wm, wn, lane, f0, 2);
    if (s == 4) read_frags_part(nxt, 0, wm, wn, lane, f0, 3);
    mma_slice<IT>(acc, f1, s);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    pend.lo[j] = lo[j];
    pend.hi[j] = hi[j];
  }
  pend.d[0] = now.pk[1].x;
  pend.d[1] = now.pk[1].y;
  pend.d[2] = now.pk[1].z;
  pend.d[3] = now.pk[1].w;
}

// Epilogue of a 16-bit output tile through LDS. Lane l holds 4 consecutive columns of one row
// per (block, group); stored to global memory straight from there, every store instruction
// writes 16 B into each of 32 rows, and measured on MI355X the 128 KiB of a 256 x 256 tile
// then take 11-16 us per tile (a GEMM with K = 3584 spent 15% of its time there). Here the
// waves first write the rounded values into LDS (free once the K loop is done: 256 rows of
// 512 B, or 448 B for 224-wide tiles, the 16-B chunks of row r XOR-swizzled by r % 32, or
// r % 4, against bank conflicts), then the threads store whole rows, 16 B per lane (a wave
// covers two rows of a 256-wide tile: 1 KiB of full 128-B lines per instruction). The arithmetic is the
// direct path's: alpha * acc, plus the bias, rounded once.
// An optional residual R added to the finished output: out = round(round(alpha * acc
// (+ bias)) + R), R [M, N] in the 16-bit output type, the two roundings of the product's own
// store followed by a separate `R + out` (a decoder layer's `residual + mlp(x)`).
struct Residual {
  const uint16_t* p;  // null: none
  int64_t ld;
};

template <int OT> QL_DEV float add_residual(float v, uint16_t r) {
  return Elem<OT>::to_f32(Elem<OT>::from_f32(v)) + Elem<OT>::to_f32(r);
}

template <int IT, int OT, int NB>
QL_DEV void tile_store_via_lds(const f32x16_t (&acc)[Layout<NB>::BI][Layout<NB>::BJ],
                               char* __restrict__ smem, typename Elem<OT>::T* __restrict__ C,
                               int64_t ldc, const uint16_t* __restrict__ bias, int64_t m0,
                               int64_t n0, int64_t M, int64_t N, float alpha, int wm, int wn,
                               int lane, const Residual& res) {
#pragma clang fp contract(off)  // alpha * acc, then + bias: two roundings, as the direct path
  using L = Layout<NB>;
  using T = typename Elem<OT>::T;
  constexpr int kChunks = 4 * NB;      // 16-B chunks of 8 values per tile row: 32 or 28
  constexpr int kRow = 16 * kChunks;   // LDS bytes per row: BM rows fit the two K-loop stages
  constexpr int kSwz = NB == 8 ? 31 : 3;  // chunk q of row r sits at q ^ (r & kSwz) < kChunks
  static_assert(BM * kRow <= 2 * stage_bytes<NB>(), "the output tile must fit the stages");
  __syncthreads();                     // every wave is done with the K loop's LDS tiles
#pragma unroll
  for (int i = 0; i < L::BI; ++i) {
    const int r = (wm * L::BI + i) * 32 + (lane & 31);
#pragma unroll
    for (int j = 0; j < L::BJ; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c = (wn * L::BJ + j) * 32 + 8 * g + 4 * (lane >> 5);  // tile column
        float v[4] = {alpha * acc[i][j][4 * g], alpha * acc[i][j][4 * g + 1],
                      alpha * acc[i][j][4 * g + 2], alpha * acc[i][j][4 * g + 3]};
        if (bias) {
          const int64_t col = n0 + c;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (col + e < N) v[e] += Elem<IT>::to_f32(bias[col + e]);
        }
        const uint32_t lo = OT == QL_BF16 ? pack_bf16x2(v[0], v[1]) : pack_f16x2(v[0], v[1]);
        const uint32_t hi = OT == QL_BF16 ? pack_bf16x2(v[2], v[3]) : pack_f16x2(v[2], v[3]);
        const int q = (c >> 3) ^ (r & kSwz);
        *reinterpret_cast<uint2*>(smem + r * kRow + q * 16 + (c & 4) * 2) = make_uint2(lo, hi);
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < BM * kChunks; idx += kThreads) {
    const int r = idx / kChunks, q = idx % kChunks;
    const int64_t row = m0 + r, col = n0 + 8 * q;
    if (row >= M || col >= N) continue;
    uint4 v = *reinterpret_cast<const uint4*>(smem + r * kRow + ((q ^ (r & kSwz)) * 16));
    T* cp = C + row * ldc + col;
    if (col + 8 <= N) {
      if (res.p) {  // the rounded product plus the residual, rounded again
        float pv[8], rv[8];
        Vec8<OT>::unpack(v, pv);
        Vec8<OT>::unpack(*reinterpret_cast<const uint4*>(res.p + row * res.ld + col), rv);
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[e] = pv[e] + rv[e];
        v = Vec8<OT>::pack(pv);
      }
      *reinterpret_cast<uint4*>(cp) = v;
    } else {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      for (int e = 0; e < 8 && col + e < N; ++e) {
        T o = (T)(w[e >> 1] >> (16 * (e & 1)));
        if (res.p)
          o = Elem<OT>::from_f32(Elem<OT>::to_f32(o) + Elem<OT>::to_f32(res.p[row * res.ld + col + e]));
        cp[e] = o;
      }
    }
  }
}

// PARTIAL: write the raw fp32 sums of this split to ws[split][M][N]; otherwise the final
// alpha / beta / bias epilogue into C (type OT). AL8: M and N are multiples of 8 and the
// loop's loads come from panels; otherwise every load clamps its rows per lane.
// K order: the second segment (A2 B2^T, K2 <= 128 columns, last split only) is loaded by the
// prologue, so every load inside the loop is a step of the first segment.
template <int IT, int OT, bool PARTIAL, int NB, bool AL8, int BQ = kBDense>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_nt_kernel(const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ B,
                    int64_t ldb, const uint16_t* __restrict__ A2, int64_t lda2,
                    const uint16_t* __restrict__ B2, int64_t ldb2, int64_t K2,
                    typename Elem<OT>::T* __restrict__ C, int64_t ldc,
                    float* __restrict__ ws, const uint16_t* __restrict__ bias, int64_t M,
                    int64_t N, int64_t K, int64_t k_per_split, float alpha, float beta,
                    bool vec_out, Nf4Operand nf4op, Residual res) {
  using L = Layout<NB>;
  constexpr bool kNf4 = BQ != kBDense;
  static_assert(!kNf4 || NB == 8, "the NF4 B operand takes 256-row tiles: one row per thread");
  constexpr int kStageBytes = stage_bytes<NB>();
  __shared__ __attribute__((aligned(1024))) char smem[2 * kStageBytes];
  __shared__ float code2_lds[BQ == kBNf4Nested ? 256 : 1];
  constexpr int BN = bn_of<NB>();
  int64_t tm, tn;
  tile_of((M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int64_t kb = (int64_t)blockIdx.y * k_per_split;
  const int64_t ke = (kb + k_per_split < K) ? kb + k_per_split : K;
  const int nk1 = (int)((ke - kb) / BK);
  // steps 0 .. nk2-1: the second segment; nk2 .. nk-1: the first (the host guarantees nk1 >= 1)
  const int nk2 = (int)blockIdx.y == (int)gridDim.y - 1 ? (int)(K2 / BK) : 0;
  const int nk = nk1 + nk2;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / L::WN, wn = wave % L::WN;

  // NF4 B: this thread's tile row, its LDS offset and swizzle, the 16 levels, code2 in LDS
  Nf4Row brow{};
  Nf4Pending pend{};
  float nf4v[16];
  uint32_t bswz = 0;
  if constexpr (kNf4) {
    const int r = threadIdx.x;
    const int64_t n = n0 + r < N ? n0 + r : N - 1;
    brow.row = nf4op.packed + n * (ldb >> 1);
    brow.w0 = n * ldb;
    bswz = (uint32_t)(((r >> 1) & 3) | ((r >> 3) & 1) << 2);
#pragma unroll
    for (int i = 0; i < 16; ++i) nf4v[i] = nf4op.nf4[i];
    if constexpr (BQ == kBNf4Nested) code2_lds[threadIdx.x] = nf4op.code2[threadIdx.x];
  }
  char* const brow_lds = smem + kATileBytes + threadIdx.x * kRowBytes;  // NF4: this thread's row

  f32x16_t acc[L::BI][L::BJ];
#pragma unroll
  for (int i = 0; i < L::BI; ++i)
#pragma unroll
    for (int j = 0; j < L::BJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  const TileLoader la = make_loader();
  if (nk > 0) {
    // prologue: steps 0 and 1, of either segment; an NF4 first-segment step's B is loaded,
    // dequantised and stored right here
    auto prologue_load = [&](int t, char* stage) {
      const bool s2 = t < nk2;
      const int64_t k0 = s2 ? (int64_t)t * BK : kb + (int64_t)(t - nk2) * BK;
      load_tile_hidden(la, s2 ? A2 : A, s2 ? lda2 : lda, m0, M, k0, stage);
      if (!kNf4 || s2) {
        load_tile_hidden<NB>(la, s2 ? B2 : B, s2 ? ldb2 : ldb, n0, N, k0, stage + kATileBytes);
      } else if constexpr (kNf4) {
        // step 1's chunks 4..7 are left to the first loop step (K2 <= 64: step 1 is NF4)
        Nf4Row now = brow;
        nf4_issue<BQ>(now, nf4op, k0);
        nf4_store_row<BQ, IT>(now, nf4op, nf4v, code2_lds, stage + (brow_lds - smem), bswz,
                              stage == smem ? nullptr : &pend);
      }
    };
    if constexpr (BQ == kBNf4Nested) __syncthreads();  // code2_lds filled
    if constexpr (!kNf4) {
      // both stages' loads go out before the first wait, which waits for stage 0 only: the
      // 8 + NB loads of stage 1 (this wave's share) may stay in flight, since loads complete
      // in issue order; the first K step's vmcnt(0) covers them before stage 1 is read
      prologue_dense<NB>(la, A, lda, B, ldb, A2, lda2, B2, ldb2, nk2, kb, m0, n0, M, N, 0, smem);
      prologue_dense<NB>(la, A, lda, B, ldb, A2, lda2, B2, ldb2, nk2, kb, m0, n0, M, N,
                         nk > 1 ? 1 : 0, smem + kStageBytes);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(8 + NB) : "memory");
      __syncthreads();
    } else {
      prologue_load(0, smem);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      prologue_load(nk > 1 ? 1 : 0, smem + kStageBytes);
    }
    if constexpr (kNf4) {  // B of loop step 0's reload target (step 2), one step ahead
      const int t2 = 2 < nk ? 2 : nk - 1;
      nf4_issue<BQ>(brow, nf4op, kb + (int64_t)(t2 - nk2) * BK);
    }
    Frags<NB> f0;
    read_frags<NB>(smem, 0, wm, wn, lane, f0);
    // loop loads: step t2 = kt + 2 (the last step reloads itself: in bounds, never read),
    // always of the first segment: k offset (t2 - nk2) * 64 from kb
    Panel<8> pa;
    Panel<NB> pb;
    if constexpr (AL8) {
      panel_init(pa, la, A, lda, m0, M, kb);
      if constexpr (!kNf4) panel_init(pb, la, B, ldb, n0, N, kb);
    }
    for (int kt = 0; kt < nk; ++kt) {
      char* cur = smem + (kt & 1) * kStageBytes;
      char* nxt = smem + ((kt + 1) & 1) * kStageBytes;
      const int t2 = kt + 2 < nk ? kt + 2 : nk - 1;
      const int q = t2 - nk2;  // >= 0: nk2 <= 2 and nk1 >= 1
      auto issue = [&](char* stage) {
        if constexpr (AL8) {
          const uint32_t kbytes = (uint32_t)q * (uint32_t)(BK * 2);
          panel_issue(pa, la, kbytes, stage);
          if constexpr (!kNf4) panel_issue(pb, la, kbytes, stage + kATileBytes);
        } else {
          const int64_t k0 = kb + (int64_t)q * BK;
          load_tile(la, A, lda, m0, M, k0, stage);
          if constexpr (!kNf4) load_tile<NB>(la, B, ldb, n0, N, k0, stage + kATileBytes);
        }
      };
      if constexpr (kNf4) {
        // B of step t2 + 1 (clamped: in bounds, never read past the last step), one step ahead
        auto issue_b = [&](Nf4Row& r) {
          const int t3 = t2 + 1 < nk ? t2 + 1 : nk - 1;
          nf4_issue<BQ>(r, nf4op, kb + (int64_t)(t3 - nk2) * BK);
        };
        mma_step_pipe_nf4<BQ, IT>(acc, f0, cur, nxt, issue, issue_b, brow, pend, nf4op, nf4v,
                                  code2_lds, (int)(brow_lds - smem), bswz, wm, wn, lane);
      } else {
        mma_step_pipe<IT, NB>(acc, f0, cur, nxt, issue, wm, wn, lane);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // 16-bit output without beta, 16-B aligned rows: the tile goes out through LDS, whole rows at
  // a time (see tile_store_via_lds); the values are those of the direct path below.
  if constexpr (!PARTIAL && OT != QL_F32) {
    if (beta == 0.f && ((uintptr_t)C & 15) == 0 && (ldc & 7) == 0) {
      tile_store_via_lds<IT, OT, NB>(acc, smem, C, ldc, bias, m0, n0, M, N, alpha, wm, wn, lane,
                                     res);
      return;
    }
  }

  // Epilogue: block (i, j) element 4g + e of lane l is row l%32, column 8g + 4(l/32) + e.
  // alpha * acc, + beta * C, + bias: each rounded to fp32 (no contraction), in both paths.
  {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < L::BI; ++i) {
    const int64_t row = m0 + (wm * L::BI + i) * 32 + (lane & 31);
    if (row >= M) continue;
#pragma unroll
    for (int j = 0; j < L::BJ; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t col = n0 + (wn * L::BJ + j) * 32 + 8 * g + 4 * (lane >> 5);
        if (col >= N) continue;
        const float a0 = acc[i][j][4 * g], a1 = acc[i][j][4 * g + 1];
        const float a2 = acc[i][j][4 * g + 2], a3 = acc[i][j][4 * g + 3];
        if constexpr (PARTIAL) {
          float* p = ws + ((int64_t)blockIdx.y * M + row) * N + col;
          if (col + 3 < N && (N & 3) == 0) {
            *reinterpret_cast<float4*>(p) = make_float4(a0, a1, a2, a3);
          } else {
            const float v[4] = {a0, a1, a2, a3};
            for (int e = 0; e < 4; ++e)
              if (col + e < N) p[e] = v[e];
          }
        } else {
          float v[4] = {alpha * a0, alpha * a1, alpha * a2, alpha * a3};
          auto* cp = C + row * ldc + col;
          if (beta != 0.f)
            for (int e = 0; e < 4; ++e)
              if (col + e < N) v[e] += beta * Elem<OT>::to_f32(cp[e]);
          if (bias)
            for (int e = 0; e < 4; ++e)
              if (col + e < N) v[e] += Elem<IT>::to_f32(bias[col + e]);
          if constexpr (OT != QL_F32) {
            if (res.p)
              for (int e = 0; e < 4; ++e)
                if (col + e < N) v[e] = add_residual<OT>(v[e], res.p[row * res.ld + col + e]);
          }
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
  }
}

// out[m, n] = alpha * sum_s ws[s][m][n] (+ beta * out) (+ bias[n]), summed in split order
// (+ the residual, after rounding); each step rounded to fp32, no contraction, as the GEMM's
// own epilogue. VW = 4: four consecutive elements of a row per thread (16-bit outputs, N and
// ldc multiples of 4, C 8-B aligned), loaded as float4 from the 16-B aligned workspace.
template <int IT, int OT>
QL_DEV uint16_t splitk_out(float s, float alpha, float beta, const uint16_t* cp,
                           const uint16_t* bias_col, const uint16_t* res_el) {
#pragma clang fp contract(off)
  float v = alpha * s;
  if (beta != 0.f) v += beta * Elem<OT>::to_f32(*cp);
  if (bias_col) v += Elem<IT>::to_f32(*bias_col);
  if (res_el) v = add_residual<OT>(v, *res_el);
  return Elem<OT>::from_f32(v);
}

template <int IT, int OT>
__global__ __launch_bounds__(256) void splitk_reduce4(const float* __restrict__ ws, int splits,
                                                      uint16_t* __restrict__ C, int64_t ldc,
                                                      const uint16_t* __restrict__ bias,
                                                      int64_t M, int64_t N, float alpha,
                                                      float beta, Residual res) {
  const int64_t total = M * N, groups = total / 4;
  for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < groups;
       g += (int64_t)gridDim.x * 256) {
    const int64_t i = 4 * g;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    int z = 0;
    for (; z + 4 <= splits; z += 4) {  // four partial vectors in flight, added in split order
      float4 w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = *reinterpret_cast<const float4*>(ws + (z + j) * total + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s[0] += w[j].x;
        s[1] += w[j].y;
        s[2] += w[j].z;
        s[3] += w[j].w;
      }
    }
    for (; z < splits; ++z) {
      const float4 w = *reinterpret_cast<const float4*>(ws + z * total + i);
      s[0] += w.x;
      s[1] += w.y;
      s[2] += w.z;
      s[3] += w.w;
    }
    const int64_t row = i / N, col = i - row * N;
    uint16_t* cp = C + row * ldc + col;
    uint16_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = splitk_out<IT, OT>(s[e], alpha, beta, cp + e, bias ? bias + col + e : nullptr,
                                res.p ? res.p + row * res.ld + col + e : nullptr);
    *reinterpret_cast<uint2*>(cp) =
        make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16));
  }
}

template <int IT, int OT>
__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ ws, int splits,
                                                     typename Elem<OT>::T* __restrict__ C,
                                                     int64_t ldc, const uint16_t* __restrict__ bias,
                                                     int64_t M, int64_t N, float alpha, float beta,
                                                     Residual res) {
#pragma clang fp contract(off)
  const int64_t total = M * N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    // 8 partials loaded at a time (independent loads in flight), added in split order
    float s = 0.f;
    int z = 0;
    for (; z + 8 <= splits; z += 8) {
      float w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) w[j] = ws[(int64_t)(z + j) * total + i];
#pragma unroll
      for (int j = 0; j < 8; ++j) s += w[j];
    }
    for (; z < splits; ++z) s += ws[(int64_t)z * total + i];
    const int64_t row = i / N, col = i - row * N;
    float v = alpha * s;
    auto* cp = C + row * ldc + col;
    if (beta != 0.f) v += beta * Elem<OT>::to_f32(*cp);
    if (bias) v += Elem<IT>::to_f32(bias[col]);
    if constexpr (OT != QL_F32) {
      if (res.p) v = add_residual<OT>(v, res.p[row * res.ld + col]);
    }
    *cp = Elem<OT>::from_f32(v);
  }
}

template <int IT, int OT, int NB, int BQ = kBDense>
int launch(const void* A, int64_t lda, const void* B, int64_t ldb, const void* A2, int64_t lda2,
           const void* B2, int64_t ldb2, int64_t K2, void* C, int64_t ldc, const void* bias,
           int64_t M, int64_t N, int64_t K, float alpha, float beta, int splits, float* ws,
           hipStream_t s, const Nf4Operand& nf4op = Nf4Operand{}, Residual res = Residual{}) {
  using T = typename Elem<OT>::T;
  constexpr int BN = bn_of<NB>();
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const int64_t kps = ((K / BK + splits - 1) / splits) * BK;
  const int nsplit = (int)((K + kps - 1) / kps);
  // panel loads: 8-row-aligned operands whose lane offsets (7 rows + K) fit in 32 bits
  constexpr int64_t kOffMax = int64_t(1) << 26;
  const bool al8 = M % 8 == 0 && N % 8 == 0 && lda < kOffMax && ldb < kOffMax && K < kOffMax;
  if (nsplit <= 1) {
    const bool vec_out = ql_aligned(C, 4 * ql_elem_size(OT)) && ldc % 4 == 0;
    if (al8)
      hipLaunchKernelGGL((gemm_nt_kernel<IT, OT, false, NB, true, BQ>), dim3((unsigned)tiles, 1),
                         dim3(kThreads), 0, s, (const uint16_t*)A, lda, (const uint16_t*)B, ldb,
                         (const uint16_t*)A2, lda2, (const uint16_t*)B2, ldb2, K2, (T*)C, ldc,
                         nullptr, (const uint16_t*)bias, M, N, K, K, alpha, beta, vec_out, nf4op,
                         res);
    else
      hipLaunchKernelGGL((gemm_nt_kernel<IT, OT, false, NB, false, BQ>), dim3((unsigned)tiles, 1),
                         dim3(kThreads), 0, s, (const uint16_t*)A, lda, (const uint16_t*)B, ldb,
                         (const uint16_t*)A2, lda2, (const uint16_t*)B2, ldb2, K2, (T*)C, ldc,
                         nullptr, (const uint16_t*)bias, M, N, K, K, alpha, beta, vec_out, nf4op,
                         res);
    return ql_launch_status();
  }
  if (al8)
    hipLaunchKernelGGL((gemm_nt_kernel<IT, QL_F32, true, NB, true, BQ>),
                       dim3((unsigned)tiles, (unsigned)nsplit), dim3(kThreads), 0, s,
                       (const uint16_t*)A, lda, (const uint16_t*)B, ldb, (const uint16_t*)A2, lda2,
                       (const uint16_t*)B2, ldb2, K2, (float*)nullptr, (int64_t)0, ws,
                       (const uint16_t*)nullptr, M, N, K, kps, 1.0f, 0.0f, false, nf4op,
                       Residual{});
  else
    hipLaunchKernelGGL((gemm_nt_kernel<IT, QL_F32, true, NB, false, BQ>),
                       dim3((unsigned)tiles, (unsigned)nsplit), dim3(kThreads), 0, s,
                       (const uint16_t*)A, lda, (const uint16_t*)B, ldb, (const uint16_t*)A2, lda2,
                       (const uint16_t*)B2, ldb2, K2, (float*)nullptr, (int64_t)0, ws,
                       (const uint16_t*)nullptr, M, N, K, kps, 1.0f, 0.0f, false, nf4op,
                       Residual{});
  int st = ql_launch_status();
  if (st != QL_OK) return st;
  const int64_t total = M * N;
  if constexpr (OT != QL_F32) {
    if (N % 4 == 0 && ldc % 4 == 0 && ((uintptr_t)C & 7) == 0) {
      int64_t grid = (total / 4 + 255) / 256;
      if (grid > 256 * 16) grid = 256 * 16;
      hipLaunchKernelGGL((splitk_reduce4<IT, OT>), dim3((unsigned)grid), dim3(256), 0, s, ws,
                         nsplit, (uint16_t*)C, ldc, (const uint16_t*)bias, M, N, alpha, beta,
                         res);
      return ql_launch_status();
    }
  }
  int64_t grid = (total + 255) / 256;
  if (grid > 256 * 16) grid = 256 * 16;
  hipLaunchKernelGGL((splitk_reduce<IT, OT>), dim3((unsigned)grid), dim3(256), 0, s, ws, nsplit,
                     (T*)C, ldc, (const uint16_t*)bias, M, N, alpha, beta, res);
  return ql_launch_status();
}

// Tile width for an M x N output: 224 when N is a multiple of 224, the output is large enough
// to run without split-K (>= 128 tiles of 256 x 256) and the narrower tiles take fewer
// (waves x tile width) on 256 CUs, else 256. The 4096 x 3584 outputs of the 7B step are 224
// tiles of 256 x 256 (one partial wave) but exactly 256 tiles of 256 x 224. Small outputs are
// split over K instead, where narrower tiles only add operand traffic.
int choose_nb(int64_t M, int64_t N) {
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

namespace {

// Split count of an M x N x K product (tile width bn): the s in 1..64 (at least 8 K steps per split) with the
// least modelled time, in units of one workgroup's K step:
//   ceil(tiles * s / 256) rounds of the 256 CUs, each (K steps per split + kTileFixedSteps)
//   long (the prologue's first load and the epilogue's stores of a tile), plus, for s > 1,
//   the split-K reduce reading s fp32 partials of the output and writing it once, at
//   kStepBytes of HBM traffic per step-time.
// An output of 192 tiles of 256 x 256 (8192 x 1536, the hidden gradient of the fused
// lm_head + CE) takes s = 4: three full rounds instead of one round on 75% of the CUs.
constexpr int64_t kCUs = 256;
constexpr int64_t kTileFixedSteps = 8;
constexpr double kStepBytes = 9.6e6;  // ~1.6 us of a K step at ~6 TB/s

int auto_splits_bn(int64_t M, int64_t N, int64_t K, int64_t bn) {
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + bn - 1) / bn);
  const int64_t steps = K / BK;
  auto cost = [&](int64_t s) {
    const int64_t rounds = (tiles * s + kCUs - 1) / kCUs;
    const double reduce = s > 1 ? double(s + 1) * double(M) * double(N) * 4.0 / kStepBytes : 0.0;
    return double(rounds * ((steps + s - 1) / s + kTileFixedSteps)) + reduce;
  };
  int best = 1;
  double best_cost = cost(1);
  for (int s = 2; s <= 64 && steps / s >= 8; ++s) {
    const double c = cost(s);
    if (c < 0.97 * best_cost) {  // a split must save at least 3% to be worth its workspace
      best = s;
      best_cost = c;
    }
  }
  return best;
}

}  // namespace

int ql_gemm_nt_auto_splits(int64_t M, int64_t N, int64_t K) {
  return auto_splits_bn(M, N, K, 32 * choose_nb(M, N));
}

int ql_gemm_nf4_auto_splits(int64_t M, int64_t N, int64_t K) {
  return auto_splits_bn(M, N, K, 256);
}

int ql_gemm_nt2(int in_dtype, int c_dtype, int64_t M, int64_t N, int64_t K, const void* A,
                int64_t lda, const void* B, int64_t ldb, const void* A2, int64_t lda2,
                const void* B2, int64_t ldb2, int64_t K2, void* C, int64_t ldc, const void* bias,
                float alpha, float beta, int splits, float* ws, hipStream_t s,
                const void* residual, int64_t ld_residual) {
  if (splits > 1 && !ws) return QL_EINVAL;
  if (residual && (c_dtype == QL_F32 || beta != 0.f || ((uintptr_t)residual & 15) ||
                   (ld_residual & 7) || ld_residual < N))
    return QL_EINVAL;
  const Residual res{static_cast<const uint16_t*>(residual), ld_residual};
  if (K2 < 0 || K2 % BK || K <= 0 || K % BK) return QL_EINVAL;
  // the kernel loads the second segment in its prologue: at most kPrologueSteps steps; the
  // sum is symmetric in the two segments, so a short first segment may take that place
  if (K2 > kPrologueSteps * BK) {
    if (K > kPrologueSteps * BK) return QL_ESHAPE;
    const void* t = A; A = A2; A2 = t;
    t = B; B = B2; B2 = t;
    int64_t u = lda; lda = lda2; lda2 = u;
    u = ldb; ldb = ldb2; ldb2 = u;
    u = K; K = K2; K2 = u;
  }
  if (K2 == 0) A2 = B2 = nullptr;
  const bool narrow = choose_nb(M, N) == 7;
#define QL_GEMM_NT_LAUNCH(ITC, NBC)                                                            \
  QL_DISPATCH_DTYPE(c_dtype, OT,                                                               \
                    return (launch<ITC, OT, NBC>(A, lda, B, ldb, A2, lda2, B2, ldb2, K2, C, ldc, \
                                                 bias, M, N, K, alpha, beta, splits, ws, s,     \
                                                 Nf4Operand{}, res)))
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

// ---- the 4-bit base GEMM: B is an NF4 weight, dequantised on its way into LDS ----------------

namespace {

int log2_exact(int64_t v) {  // log2 of a power of two, else -1
  if (v <= 0 || (v & (v - 1))) return -1;
  int l = 0;
  while ((int64_t(1) << l) < v) ++l;
  return l;
}

}  // namespace

extern "C" int64_t qlora_gemm_nf4_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % BK) return 0;
  return ql_gemm_nt_workspace_floats(M, N, ql_gemm_nf4_auto_splits(M, N, K)) *
         (int64_t)sizeof(float);
}

extern "C" int qlora_gemm_nf4(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                              const uint8_t* packed, const void* absmax, int nested,
                              const float* code2, const float* absmax2, float offset,
                              int blocksize, int blocksize2, const float* nf4_table, int64_t K2,
                              const void* A2, int64_t lda2, const void* B2, int64_t ldb2,
                              int in_dtype, void* C, int64_t ldc, const void* bias, float alpha,
                              void* workspace, int64_t workspace_bytes, ql_stream_t stream) {
  if (M < 0 || N < 0 || K < 0 || K2 < 0 || workspace_bytes < 0) return QL_EINVAL;
  if (in_dtype != QL_BF16 && in_dtype != QL_F16) return QL_EDTYPE;
  if (M == 0 || N == 0) return QL_OK;
  if (!A || !packed || !absmax || !nf4_table || !C) return QL_EINVAL;
  if (nested && (!code2 || !absmax2)) return QL_EINVAL;
  if (K2 > 0 && (!A2 || !B2)) return QL_EINVAL;
  // the LoRA segment takes one prologue step, so prologue step 1 is always an NF4 step
  if (K <= 0 || K % BK || K2 % BK || K2 > BK) return QL_ESHAPE;
  const int log2_bs = log2_exact(blocksize);
  const int log2_bs2 = nested ? log2_exact(blocksize2) : 0;
  if (log2_bs < 6 || K % blocksize || log2_bs2 < 0) return QL_EINVAL;
  if (lda < K || ldc < N || (K2 > 0 && (lda2 < K2 || ldb2 < K2))) return QL_ESHAPE;
  if (lda % 8 || !ql_aligned(A, 16) || !ql_aligned(packed, 16) || !ql_aligned(C, 2) ||
      (bias && !ql_aligned(bias, 2)))
    return QL_EALIGN;
  if (K2 > 0 && !ql_gemm_nt_fits(M, N, K2, A2, lda2, B2, ldb2)) return QL_EALIGN;
  if ((M + BM - 1) / BM * ((N + 255) / 256) >= (int64_t(1) << 30)) return QL_ESHAPE;
  int splits = ql_gemm_nf4_auto_splits(M, N, K);
  const int64_t need = ql_gemm_nt_workspace_floats(M, N, splits) * (int64_t)sizeof(float);
  if (need > workspace_bytes || !workspace || !ql_aligned(workspace, 16)) splits = 1;
  const Nf4Operand op{packed, absmax, absmax2, code2, nf4_table, offset, log2_bs, log2_bs2};
  float* ws = static_cast<float*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (K2 == 0) A2 = B2 = nullptr;
  // B's leading dimension is K: the weight's row length, in weights
#define QL_NF4_LAUNCH(ITC, BQC)                                                                \
  return launch<ITC, ITC, 8, BQC>(A, lda, nullptr, K, A2, lda2, B2, ldb2, K2, C, ldc, bias, M, \
                                  N, K, alpha, 0.f, splits, ws, s, op)
  if (in_dtype == QL_BF16) {
    if (nested) QL_NF4_LAUNCH(QL_BF16, kBNf4Nested);
    QL_NF4_LAUNCH(QL_BF16, kBNf4Plain);
  }
  if (nested) QL_NF4_LAUNCH(QL_F16, kBNf4Nested);
  QL_NF4_LAUNCH(QL_F16, kBNf4Plain);
#undef QL_NF4_LAUNCH
}

// ---------------------------------------------------------------------------------------------
// The matrix-core rate with no memory traffic: each wave of one 4-wave workgroup per CU (one
// wave per SIMD, as the GEMM runs) issues the GEMM's inner product pattern, a 4 x 4 grid of
// v_mfma_f32_32x32x16 into 16 accumulators, twice per round (two fragment sets), `iters`
// rounds. Mode 0 keeps both sets of 4 A and 4 B fragments of the given data in registers; mode
// 1 reads every set's 8 fragments from a 64 KiB LDS tile of that data (one ds_read_b128 each,
// conflict-free, the next set's reads issued before the current set's products), the GEMM's
// fragment traffic without its global loads; mode 2 adds the GEMM's K-loop pipeline (two 64 KiB
// stages, one barrier and 16 direct-to-LDS loads of 1 KiB per wave per 64-k step, from a 2 MiB
// source that stays in L2), without tile edges or output; mode 3 is mode 2 with those loads
// staged through registers (global_load_dwordx4, then ds_write_b128 after the step's products).
// The rate on N(0,1) against all-zero
// operands is the power/clock ceiling of this part for that data; each mode against the one
// before is what that layer of the GEMM's pipeline costs. Measurement only; nothing in the
// QLoRA step calls it.
namespace {

constexpr int kProbeTile = 4096;  // uint4 in the mode-1 LDS tile (64 KiB)
typedef int probe_v4_t __attribute__((ext_vector_type(4)));
constexpr int64_t kProbeSrcBytes = 2 << 20;  // mode-2 source: 2 MiB, resident in each XCD's L2

template <int DT, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void mfma_probe_kernel(const uint4* __restrict__ ops, int64_t iters, float* __restrict__ out,
                       const char* __restrict__ src) {
  __shared__ __attribute__((aligned(1024))) uint4 tile[MODE == 0 ? 1 : MODE == 1 ? kProbeTile
                                                                                : 2 * kProbeTile];
  const int lane = threadIdx.x & 63;
  f32x16_t acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x16_t{};
  if constexpr (MODE == 0) {
    uint4 a[2][4], b[2][4];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[s][i] = ops[(s * 8 + i) * 64 + lane];
        b[s][i] = ops[(s * 8 + 4 + i) * 64 + lane];
      }
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[4 * i + j] = mfma<DT>(a[s][i], b[s][j], acc[4 * i + j]);
    }
  } else if constexpr (MODE == 2) {
    // the GEMM's K loop without its tile edges: two 64 KiB stages; per 64-k step every wave
    // waits for the step's loads, meets the others at one barrier, issues 16 direct-to-LDS
    // loads of 1 KiB into the other stage (from the L2-resident source; workgroups start at
    // different 64 KiB windows of it, as the GEMM's tiles read different rows) and runs 4
    // sub-steps of 8 fragment reads and 16 products on this stage
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for (int t = threadIdx.x; t < kProbeTile; t += 256) tile[t] = ops[t % 1024];
    const int64_t steps = iters / 2 > 0 ? iters / 2 : 1;  // 64 products a wave per step
    for (int64_t st = 0; st < steps; ++st) {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const uint4* cur = tile + (st & 1) * kProbeTile;
      char* nxt = reinterpret_cast<char*>(tile + ((st + 1) & 1) * kProbeTile);
      const int64_t soff = ((st + 1 + blockIdx.x) * 65536 + wave * 16384) % kProbeSrcBytes;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        dma_hidden(src + soff + j * 1024, (uint32_t)(lane * 16), nxt + wave * 16384 + j * 1024);
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        uint4 a[4], b[4];
        const int base = sub * 1024 + lane;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = cur[base + 64 * i];
          b[i] = cur[base + 64 * (4 + i)];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[4 * i + j] = mfma<DT>(a[i], b[j], acc[4 * i + j]);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else if constexpr (MODE == 3) {
    // mode 2 with the loads staged through registers: 16 global_load_dwordx4 per wave at the
    // step's start, written to the other stage with ds_write_b128 after the step's products
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for (int t = threadIdx.x; t < kProbeTile; t += 256) tile[t] = ops[t % 1024];
    const int64_t steps = iters / 2 > 0 ? iters / 2 : 1;
    for (int64_t st = 0; st < steps; ++st) {
      __syncthreads();
      const uint4* cur = tile + (st & 1) * kProbeTile;
      uint4* nxt = tile + ((st + 1) & 1) * kProbeTile;
      const int64_t soff = ((st + 1 + blockIdx.x) * 65536 + wave * 16384) % kProbeSrcBytes;
      const uint4* sp = reinterpret_cast<const uint4*>(src + soff);
      // the loads go out before the products and are waited for only before their stores
      // (as inline assembly: left to itself the compiler sinks them to the stores)
      probe_v4_t stage[16];
#pragma unroll
      for (int j = 0; j < 16; ++j)
        asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(stage[j]) : "v"(sp + j * 64 + lane));
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        uint4 a[4], b[4];
        const int base = sub * 1024 + lane;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = cur[base + 64 * i];
          b[i] = cur[base + 64 * (4 + i)];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[4 * i + j] = mfma<DT>(a[i], b[j], acc[4 * i + j]);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int j = 0; j < 16; ++j)
        nxt[wave * 1024 + j * 64 + lane] = __builtin_bit_cast(uint4, stage[j]);
    }
  } else {
    for (int t = threadIdx.x; t < kProbeTile; t += 256) tile[t] = ops[t % 1024];
    __syncthreads();
    // set n reads 8 fragments of 1 KiB (64 lanes x 16 B, contiguous) from 8 KiB slice n % 8
    auto load_set = [&](int64_t n, uint4* a, uint4* b) {
      const int base = (int)(n & 7) * 512 + lane;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = tile[base + 64 * i];
        b[i] = tile[base + 64 * (4 + i)];
      }
    };
    uint4 a[4], b[4], an[4], bn[4];
    load_set(0, a, b);
    for (int64_t n = 0; n < 2 * iters; ++n) {
      load_set(n + 1, an, bn);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[4 * i + j] = mfma<DT>(a[i], b[j], acc[4 * i + j]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = an[i];
        b[i] = bn[i];
      }
    }
  }
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) t += acc[i][e];
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = t;
}

}  // namespace

extern "C" int qlora_mfma_probe(const void* operands, int dtype, int mode, int64_t iters,
                                int workgroups, float* out, const void* source,
                                ql_stream_t stream) {
  if (!operands || !out || iters <= 0 || workgroups <= 0 || workgroups > 65535) return QL_EINVAL;
  if (mode < 0 || mode > 3 || (mode >= 2 && (!source || !ql_aligned(source, 16))))
    return QL_EINVAL;
  if (dtype != QL_BF16 && dtype != QL_F16) return QL_EDTYPE;
  if (!ql_aligned(operands, 16)) return QL_EALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define QL_PROBE(DTC, MC)                                                                      \
  hipLaunchKernelGGL((mfma_probe_kernel<DTC, MC>), dim3(workgroups), dim3(256), 0, s,          \
                     (const uint4*)operands, iters, out, (const char*)source)
  if (dtype == QL_BF16) {
    if (mode == 0) QL_PROBE(QL_BF16, 0);
    else if (mode == 1) QL_PROBE(QL_BF16, 1);
    else if (mode == 2) QL_PROBE(QL_BF16, 2);
    else QL_PROBE(QL_BF16, 3);
  } else {
    if (mode == 0) QL_PROBE(QL_F16, 0);
    else if (mode == 1) QL_PROBE(QL_F16, 1);
    else if (mode == 2) QL_PROBE(QL_F16, 2);
    else QL_PROBE(QL_F16, 3);
  }
#undef QL_PROBE
  return ql_launch_status();
}
