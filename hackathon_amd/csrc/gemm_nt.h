// Internal interface of the large-tile NT GEMM (gemm_nt.hip), used by the C-ABI entry points
// of gemm.hip and by the fused layers. Not part of the public C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// True when the NT kernel takes this problem: K % 64 == 0, lda and ldb multiples of 8
// elements, A and B 16-B aligned.
bool ql_gemm_nt_fits(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* B,
                     int64_t ldb);

// Split count that fills 256 CUs for this shape (1 = no split-K).
int ql_gemm_nt_auto_splits(int64_t M, int64_t N, int64_t K);

// fp32 elements of workspace ql_gemm_nt needs with `splits` splits (0 when splits <= 1).
int64_t ql_gemm_nt_workspace_floats(int64_t M, int64_t N, int splits);

// C = alpha * A @ B^T (+ beta C) (+ bias); ws must hold ql_gemm_nt_workspace_floats floats
// (16-B aligned) when splits > 1.
int ql_gemm_nt(int in_dtype, int c_dtype, int64_t M, int64_t N, int64_t K, const void* A,
               int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, const void* bias,
               float alpha, float beta, int splits, float* ws, hipStream_t s);

// C = alpha * (A @ B^T + A2 @ B2^T) (+ beta C) (+ bias): a second k-contiguous segment with
// K2 % 64 == 0 columns (A2 [M, K2], B2 [N, K2], same alignment rules; K2 = 0: none). With
// `residual` (16-bit C only, beta 0; [M, N] in C's type, 16-B aligned rows, ld % 8 == 0) the
// rounded result plus the residual, rounded again.
int ql_gemm_nt2(int in_dtype, int c_dtype, int64_t M, int64_t N, int64_t K, const void* A,
                int64_t lda, const void* B, int64_t ldb, const void* A2, int64_t lda2,
                const void* B2, int64_t ldb2, int64_t K2, void* C, int64_t ldc, const void* bias,
                float alpha, float beta, int splits, float* ws, hipStream_t s,
                const void* residual = nullptr, int64_t ld_residual = 0);
