// Dense bf16/fp16 GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x32_{bf16,f16}).
//
//   C[M,N] = alpha * sum_k A[m,k] * B[n,k]  (+ beta * C) (+ bias[n])
//
// Operand storage (template flags):
//   A: "MK" (row m at A + m*lda, k contiguous)   or "KM" (k at A + k*lda, m contiguous)
//   B: "NK" (row n at B + n*ldb, k contiguous)   or "KN" (k at B + k*ldb, n contiguous)
// so one kernel serves x @ W^T (A MK, B NK), dY @ W (A MK, B KN) and dY^T @ U (A KM, B KN).
// These replace the torch GEMM call sites of the reference: solution/nf4.py:102,111,
// solution/lora.py:172, solution/cross_entropy.py:117,123, solution/fused_ce.py:135,143.
//
// Tiling for gfx950 (256 CUs, wave64, 160 KiB LDS per CU):
//   workgroup tile 128 x 128 x 64, 256 threads = 4 waves in a 2 x 2 grid of 64 x 64;
//   each wave holds 4 x 4 MFMA 16x16 accumulators (64 fp32 VGPRs).
//   LDS holds both operands K-contiguous ([row][k], rows padded by 16 B so the 8 lanes of
//   each ds_read_b128 phase hit distinct banks), double-buffered: the global loads of tile
//   k+1 are in flight while tile k is multiplied, then written to the other buffer; one
//   barrier per K step.
//   Operands stored K-outer ("KM"/"KN") are transposed in registers on their way to LDS:
//   a thread loads an 8(k) x 4(row) block with 8-byte loads and writes 4 rows of 8 k.
//   The MFMA is issued with the B fragment as its first operand, so each lane ends up owning
//   one output row and 4 consecutive output columns: the epilogue stores 8 B (bf16) or 16 B
//   (fp32) per lane per 16x16 tile.
#include "ql_vec.h"
#include "gemm_nt.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kThreads = 256;
constexpr int LDS_ROW = BK + 8;             // padded row, in 16-bit elements (144 B)
constexpr int LDS_TILE = 128 * LDS_ROW;     // one operand tile, in elements

template <int DT> QL_DEV f32x4_t mfma16(const uint4& a, const uint4& b, f32x4_t c);
template <> QL_DEV f32x4_t mfma16<QL_BF16>(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <> QL_DEV f32x4_t mfma16<QL_F16>(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Staging registers of one operand tile (128 rows x 64 k) for one thread: 64 B.
struct Stage {
  uint4 v[4];
};

// ---- operand stored [rows, K] (k contiguous): thread owns 16-B chunks tid + 256*i ----------
// `vec`: rows are 16-B aligned (ld % 8 == 0, base aligned), so an in-range chunk is one 16-B
// load; chunks crossing K (or unaligned rows) are loaded element by element, zero past K.
QL_DEV void load_rk(Stage& st, const uint16_t* __restrict__ X, int64_t ld, int64_t r0, int64_t k0,
                    int64_t R, int64_t K, bool vec) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + kThreads * i;
    const int r = c >> 3, kc = (c & 7) * 8;
    const int64_t gr = r0 + r, gk = k0 + kc;
    if (gr < R && vec && gk + 8 <= K) {
      st.v[i] = *reinterpret_cast<const uint4*>(X + gr * ld + gk);
    } else if (gr < R && gk < K) {
      uint32_t w[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t lo = (gk + 2 * p < K) ? X[gr * ld + gk + 2 * p] : 0u;
        const uint32_t hi = (gk + 2 * p + 1 < K) ? X[gr * ld + gk + 2 * p + 1] : 0u;
        w[p] = lo | (hi << 16);
      }
      st.v[i] = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      st.v[i] = make_uint4(0, 0, 0, 0);
    }
  }
}

QL_DEV void store_rk(const Stage& st, uint16_t* lds) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + kThreads * i;
    const int r = c >> 3, kc = (c & 7) * 8;
    *reinterpret_cast<uint4*>(lds + r * LDS_ROW + kc) = st.v[i];
  }
}

// ---- operand stored [K, rows] (rows contiguous): thread owns an 8(k) x 4(row) block --------
// kb = tid / 32 selects k rows 8kb..8kb+7, rb = tid % 32 selects rows 4rb..4rb+3.
QL_DEV void load_kr(Stage& st, const uint16_t* __restrict__ X, int64_t ld, int64_t r0, int64_t k0,
                    int64_t R, int64_t K, bool vec) {
  const int kb = threadIdx.x >> 5, rb = threadIdx.x & 31;
  const int64_t gr = r0 + 4 * rb;
  uint2 in[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const int64_t gk = k0 + 8 * kb + kk;
    if (gk < K && vec && gr + 3 < R) {
      in[kk] = *reinterpret_cast<const uint2*>(X + gk * ld + gr);  // 8-B aligned (host check)
    } else if (gk < K && gr < R) {
      uint16_t e[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) e[j] = (gr + j < R) ? X[gk * ld + gr + j] : (uint16_t)0;
      in[kk] = make_uint2((uint32_t)e[0] | ((uint32_t)e[1] << 16), (uint32_t)e[2] | ((uint32_t)e[3] << 16));
    } else {
      in[kk] = make_uint2(0, 0);
    }
  }
  // transpose 8 x 4 (k x row) into 4 rows of 8 k (packed pairs along k)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t a = (r < 2) ? in[2 * p].x : in[2 * p].y;
      const uint32_t b = (r < 2) ? in[2 * p + 1].x : in[2 * p + 1].y;
      w[p] = (r & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
    st.v[r] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

QL_DEV void store_kr(const Stage& st, uint16_t* lds) {
  const int kb = threadIdx.x >> 5, rb = threadIdx.x & 31;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    *reinterpret_cast<uint4*>(lds + (4 * rb + r) * LDS_ROW + 8 * kb) = st.v[r];
}

template <bool KMAJOR>
QL_DEV void load_op(Stage& st, const uint16_t* X, int64_t ld, int64_t r0, int64_t k0, int64_t R,
                    int64_t K, bool vec) {
  if constexpr (KMAJOR) load_kr(st, X, ld, r0, k0, R, K, vec);
  else load_rk(st, X, ld, r0, k0, R, K, vec);
}

template <bool KMAJOR>
QL_DEV void store_op(const Stage& st, uint16_t* lds) {
  if constexpr (KMAJOR) store_kr(st, lds);
  else store_rk(st, lds);
}

template <int OT>
QL_DEV void store4(typename Elem<OT>::T* p, const float* v, bool vec) {
  if constexpr (OT == QL_F32) {
    if (vec) *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    else for (int j = 0; j < 4; ++j) p[j] = v[j];
  } else {
    if (vec) {
      uint2 w;
      if constexpr (OT == QL_BF16) w = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      else w = make_uint2(pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3]));
      *reinterpret_cast<uint2*>(p) = w;
    } else {
      for (int j = 0; j < 4; ++j) p[j] = Elem<OT>::from_f32(v[j]);
    }
  }
}

template <int IT, bool A_KM, bool B_KN, int OT>
__global__ __launch_bounds__(kThreads, 2) void gemm_mfma_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ B, int64_t ldb,
    typename Elem<OT>::T* __restrict__ C, int64_t ldc, const uint16_t* __restrict__ bias,
    int64_t M, int64_t N, int64_t K, float alpha, float beta, bool vec_a, bool vec_b,
    bool vec_out) {
  // LDS: [A buf0 | B buf0 | A buf1 | B buf1], each LDS_TILE elements
  extern __shared__ uint16_t smem[];

  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = (int64_t)blockIdx.x * BN;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 15;        // fragment row within a 16-row sub-tile
  const int lk = (lane >> 4) * 8;  // fragment k offset within a 32-k step

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int64_t nk = (K + BK - 1) / BK;
  Stage sa, sb;
  load_op<A_KM>(sa, A, lda, m0, 0, M, K, vec_a);
  load_op<B_KN>(sb, B, ldb, n0, 0, N, K, vec_b);
  store_op<A_KM>(sa, smem);
  store_op<B_KN>(sb, smem + LDS_TILE);
  __syncthreads();

  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      load_op<A_KM>(sa, A, lda, m0, (kt + 1) * BK, M, K, vec_a);
      load_op<B_KN>(sb, B, ldb, n0, (kt + 1) * BK, N, K, vec_b);
    }
    const uint16_t* as = smem + cur * 2 * LDS_TILE + (wm * 64 + lr) * LDS_ROW + lk;
    const uint16_t* bs = smem + cur * 2 * LDS_TILE + LDS_TILE + (wn * 64 + lr) * LDS_ROW + lk;
#pragma unroll
    for (int ks = 0; ks < BK; ks += 32) {
      uint4 af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<const uint4*>(as + i * 16 * LDS_ROW + ks);
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = *reinterpret_cast<const uint4*>(bs + j * 16 * LDS_ROW + ks);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<IT>(bf[j], af[i], acc[i][j]);
    }
    if (more) {
      store_op<A_KM>(sa, smem + (cur ^ 1) * 2 * LDS_TILE);
      store_op<B_KN>(sb, smem + (cur ^ 1) * 2 * LDS_TILE + LDS_TILE);
    }
    __syncthreads();
  }

  // epilogue: lane owns row (lane & 15) and columns 4*(lane >> 4) .. +3 of each 16x16 tile
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = m0 + wm * 64 + i * 16 + lr;
    if (row >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + wn * 64 + j * 16 + (lane >> 4) * 4;
      if (col >= N) continue;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = alpha * acc[i][j][e];
      auto* cp = C + row * ldc + col;
      const bool full = col + 3 < N;
      if (beta != 0.f) {
        for (int e = 0; e < 4; ++e)
          if (col + e < N) v[e] += beta * Elem<OT>::to_f32(cp[e]);
      }
      if (bias) {
        for (int e = 0; e < 4; ++e)
          if (col + e < N) v[e] += Elem<IT>::to_f32(bias[col + e]);
      }
      if (full) {
        store4<OT>(cp, v, vec_out);
      } else {
        for (int e = 0; e < 4; ++e)
          if (col + e < N) cp[e] = Elem<OT>::from_f32(v[e]);
      }
    }
  }
}

constexpr size_t kSmemBytes = 4 * LDS_TILE * sizeof(uint16_t);  // 2 buffers x (A + B)

template <int IT, bool A_KM, bool B_KN, int OT>
int launch(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
           const void* bias, int64_t M, int64_t N, int64_t K, float alpha, float beta,
           hipStream_t s) {
  auto kern = gemm_mfma_kernel<IT, A_KM, B_KN, OT>;
  static bool attr_set = false;  // per instantiation; the attribute is per function
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSmemBytes);
    if (e != hipSuccess) return ql_hip_status(e);
    attr_set = true;
  }
  const int64_t esz = ql_elem_size(OT);
  const bool vec_out = ql_aligned(C, 4 * esz) && ((ldc * esz) % (4 * esz)) == 0;
  // vector operand loads: 16 B along k for k-contiguous operands, 8 B along rows otherwise
  const bool vec_a = A_KM ? (ql_aligned(A, 8) && lda % 4 == 0) : (ql_aligned(A, 16) && lda % 8 == 0);
  const bool vec_b = B_KN ? (ql_aligned(B, 8) && ldb % 4 == 0) : (ql_aligned(B, 16) && ldb % 8 == 0);
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), kSmemBytes, s, (const uint16_t*)A, lda,
                     (const uint16_t*)B, ldb, (typename Elem<OT>::T*)C, ldc, (const uint16_t*)bias,
                     M, N, K, alpha, beta, vec_a, vec_b, vec_out);
  return ql_launch_status();
}

template <int IT, int OT>
int dispatch_layout(int a_km, int b_kn, const void* A, int64_t lda, const void* B, int64_t ldb,
                    void* C, int64_t ldc, const void* bias, int64_t M, int64_t N, int64_t K,
                    float alpha, float beta, hipStream_t s) {
  if (!a_km && !b_kn) return launch<IT, false, false, OT>(A, lda, B, ldb, C, ldc, bias, M, N, K, alpha, beta, s);
  if (!a_km && b_kn) return launch<IT, false, true, OT>(A, lda, B, ldb, C, ldc, bias, M, N, K, alpha, beta, s);
  if (a_km && b_kn) return launch<IT, true, true, OT>(A, lda, B, ldb, C, ldc, bias, M, N, K, alpha, beta, s);
  return launch<IT, true, false, OT>(A, lda, B, ldb, C, ldc, bias, M, N, K, alpha, beta, s);
}

}  // namespace

namespace {

int gemm_checked(int a_km, int b_kn, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                 const void* B, int64_t ldb, int in_dtype, void* C, int64_t ldc, int c_dtype,
                 const void* bias, float alpha, float beta, void* ws, int64_t ws_bytes,
                 hipStream_t s) {
  if (M < 0 || N < 0 || K < 0 || ws_bytes < 0) return QL_EINVAL;
  if (in_dtype != QL_BF16 && in_dtype != QL_F16) return QL_EDTYPE;
  if (!ql_valid_dtype(c_dtype)) return QL_EDTYPE;
  if (M == 0 || N == 0) return QL_OK;
  if (!C || (K > 0 && (!A || !B))) return QL_EINVAL;
  if (M > (int64_t)65535 * BM || N > (int64_t)INT32_MAX) return QL_EINVAL;
  if (!ql_aligned(A, 2) || !ql_aligned(B, 2) || !ql_aligned(C, ql_elem_size(c_dtype)))
    return QL_EALIGN;
  if (lda < (a_km ? M : K) || ldb < (b_kn ? N : K) || ldc < N) return QL_ESHAPE;
  if (!a_km && !b_kn && ql_gemm_nt_fits(M, N, K, A, lda, B, ldb)) {
    int splits = ql_gemm_nt_auto_splits(M, N, K);
    const int64_t need = ql_gemm_nt_workspace_floats(M, N, splits) * (int64_t)sizeof(float);
    if (need > ws_bytes || !ws || !ql_aligned(ws, 16)) splits = 1;
    return ql_gemm_nt(in_dtype, c_dtype, M, N, K, A, lda, B, ldb, C, ldc, bias, alpha, beta,
                      splits, static_cast<float*>(ws), s);
  }
  if (in_dtype == QL_BF16) {
    QL_DISPATCH_DTYPE(c_dtype, OT,
                      return dispatch_layout<QL_BF16, OT>(a_km, b_kn, A, lda, B, ldb, C, ldc, bias,
                                                          M, N, K, alpha, beta, s));
  } else {
    QL_DISPATCH_DTYPE(c_dtype, OT,
                      return dispatch_layout<QL_F16, OT>(a_km, b_kn, A, lda, B, ldb, C, ldc, bias,
                                                         M, N, K, alpha, beta, s));
  }
  return QL_EDTYPE;
}

}  // namespace

extern "C" int qlora_gemm(int a_km, int b_kn, int64_t M, int64_t N, int64_t K, const void* A,
                          int64_t lda, const void* B, int64_t ldb, int in_dtype, void* C,
                          int64_t ldc, int c_dtype, const void* bias, float alpha, float beta,
                          ql_stream_t stream) {
  return gemm_checked(a_km, b_kn, M, N, K, A, lda, B, ldb, in_dtype, C, ldc, c_dtype, bias, alpha,
                      beta, nullptr, 0, static_cast<hipStream_t>(stream));
}

extern "C" int64_t qlora_gemm_workspace_size(int a_km, int b_kn, int64_t M, int64_t N,
                                             int64_t K) {
  if (a_km || b_kn || M <= 0 || N <= 0 || K <= 0 || K % 64) return 0;
  return ql_gemm_nt_workspace_floats(M, N, ql_gemm_nt_auto_splits(M, N, K)) *
         (int64_t)sizeof(float);
}

extern "C" int qlora_gemm_ws(int a_km, int b_kn, int64_t M, int64_t N, int64_t K, const void* A,
                             int64_t lda, const void* B, int64_t ldb, int in_dtype, void* C,
                             int64_t ldc, int c_dtype, const void* bias, float alpha, float beta,
                             void* workspace, int64_t workspace_bytes, ql_stream_t stream) {
  return gemm_checked(a_km, b_kn, M, N, K, A, lda, B, ldb, in_dtype, C, ldc, c_dtype, bias, alpha,
                      beta, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int64_t qlora_gemm_nt_cat_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K < 0 || K % 64) return 0;
  return ql_gemm_nt_workspace_floats(M, N, ql_gemm_nt_auto_splits(M, N, K)) *
         (int64_t)sizeof(float);
}

static int gemm_nt_cat(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                       const void* B, int64_t ldb, int64_t K2, const void* A2, int64_t lda2,
                       const void* B2, int64_t ldb2, int in_dtype, void* C, int64_t ldc,
                       int c_dtype, const void* bias, float alpha, const void* residual,
                       int64_t ld_residual, void* workspace, int64_t workspace_bytes,
                       ql_stream_t stream) {
  if (M < 0 || N < 0 || K < 0 || K2 < 0 || workspace_bytes < 0) return QL_EINVAL;
  if (in_dtype != QL_BF16 && in_dtype != QL_F16) return QL_EDTYPE;
  if (!ql_valid_dtype(c_dtype)) return QL_EDTYPE;
  if (M == 0 || N == 0) return QL_OK;
  if (!C || (K > 0 && (!A || !B)) || (K2 > 0 && (!A2 || !B2))) return QL_EINVAL;
  if (K % 64 || K2 % 64 || K + K2 == 0) return QL_ESHAPE;
  if (lda < K || ldb < K || ldc < N || (K2 > 0 && (lda2 < K2 || ldb2 < K2))) return QL_ESHAPE;
  if (!ql_aligned(C, ql_elem_size(c_dtype))) return QL_EALIGN;
  if (K > 0 && !ql_gemm_nt_fits(M, N, K, A, lda, B, ldb)) return QL_EALIGN;
  if (K2 > 0 && !ql_gemm_nt_fits(M, N, K2, A2, lda2, B2, ldb2)) return QL_EALIGN;
  if (K == 0) {  // the second segment alone
    A = A2; lda = lda2; B = B2; ldb = ldb2; K = K2; K2 = 0; A2 = B2 = nullptr;
  }
  int splits = ql_gemm_nt_auto_splits(M, N, K);
  const int64_t need = ql_gemm_nt_workspace_floats(M, N, splits) * (int64_t)sizeof(float);
  if (need > workspace_bytes || !workspace || !ql_aligned(workspace, 16)) splits = 1;
  if (residual) {
    if (c_dtype == QL_F32) return QL_EDTYPE;
    if (ld_residual < N) return QL_ESHAPE;
    if (!ql_aligned(residual, 16) || ld_residual % 8) return QL_EALIGN;
    // the residual is read while the output is written: no overlap
    const char* r0 = static_cast<const char*>(residual);
    const char* c0 = static_cast<const char*>(C);
    const int64_t rbytes = ((M - 1) * ld_residual + N) * 2, cbytes = ((M - 1) * ldc + N) * 2;
    if (r0 < c0 + cbytes && c0 < r0 + rbytes) return QL_EINVAL;
  }
  return ql_gemm_nt2(in_dtype, c_dtype, M, N, K, A, lda, B, ldb, A2, lda2, B2, ldb2, K2, C, ldc,
                     bias, alpha, 0.f, splits, static_cast<float*>(workspace),
                     static_cast<hipStream_t>(stream), residual, ld_residual);
}

extern "C" int qlora_gemm_nt_cat(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                                 const void* B, int64_t ldb, int64_t K2, const void* A2,
                                 int64_t lda2, const void* B2, int64_t ldb2, int in_dtype, void* C,
                                 int64_t ldc, int c_dtype, const void* bias, float alpha,
                                 void* workspace, int64_t workspace_bytes, ql_stream_t stream) {
  return gemm_nt_cat(M, N, K, A, lda, B, ldb, K2, A2, lda2, B2, ldb2, in_dtype, C, ldc, c_dtype,
                     bias, alpha, nullptr, 0, workspace, workspace_bytes, stream);
}

extern "C" int qlora_gemm_nt_cat_residual(int64_t M, int64_t N, int64_t K, const void* A,
                                          int64_t lda, const void* B, int64_t ldb, int64_t K2,
                                          const void* A2, int64_t lda2, const void* B2,
                                          int64_t ldb2, int in_dtype, void* C, int64_t ldc,
                                          int c_dtype, const void* residual, int64_t ld_residual,
                                          void* workspace, int64_t workspace_bytes,
                                          ql_stream_t stream) {
  if (!residual) return QL_EINVAL;
  return gemm_nt_cat(M, N, K, A, lda, B, ldb, K2, A2, lda2, B2, ldb2, in_dtype, C, ldc, c_dtype,
                     nullptr, 1.0f, residual, ld_residual, workspace, workspace_bytes, stream);
}
