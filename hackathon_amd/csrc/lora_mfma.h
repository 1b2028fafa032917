// Internal interface of the rank-16 LoRA MFMA kernels (lora_mfma.hip). Not part of the
// public C-ABI; the C-ABI entry points at the end of lora_mfma.hip call these.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// For `slots` = G (1 .. 4) adapters that share X: out[m, c] = alpha * sum_k X[m, k] Y[c, k]
// for c < 16 G (Y [16 G, K], slot g in rows 16 g .. 16 g + 15), zeros for 16 G <= c <
// out_cols, and (out_t not null) the same 16 G columns transposed into out_t [16 G, ldt >= M]
// in the input dtype. K % 32 == 0; X, Y 16-B aligned with ldx, ldy multiples of 8 and
// 32 ldx, 32 G ldy < 2^31. ws (fp32, may be null) lets the K reduction split over more
// workgroups.
int ql_lora_down(int in_dtype, int out_dtype, const void* X, int64_t ldx, const void* Y,
                 int64_t ldy, int64_t M, int64_t K, int slots, void* out, int64_t ldo,
                 int out_cols, float alpha, void* out_t, int64_t ldt, float* ws,
                 int64_t ws_floats, hipStream_t s);
int64_t ql_lora_down_workspace_floats(int64_t M, int64_t K, int slots);

// The dropout masks of the lora_A gradients over one shared input: adapter g's products use
// keep_g * (Q * scale rounded to Q's type) in place of Q, keep_g from its bits (the 8 x 8
// block layout of ql_philox.h, 8-B aligned, group stride gs: a multiple of 8, >= N).
struct WgradMask {
  const uint8_t* p[4];
  int64_t gs;
  float scale;
};

// out[n, c] = alpha * sum_m Q[m, n] PT[c, m] for c < 16 G (fp32 [N, 16 G], 16-B aligned).
// N % 8 == 0; Q 16-B aligned with ldq a multiple of 8, 64 ldq < 2^31; PT [16 G, ldpt >= M]
// (P transposed, token-contiguous), 16-B aligned with ldpt a multiple of 8, 32 G ldpt < 2^31.
// out_t = 1 stores out transposed, [16 G, N]. With `mask`, Q is each adapter's dropped input.
int ql_lora_wgrad(int in_dtype, const void* PT, int64_t ldpt, const void* Q, int64_t ldq,
                  int64_t M, int64_t N, int slots, float* out, int out_t, float alpha, float* ws,
                  int64_t ws_floats, hipStream_t s, const WgradMask* mask = nullptr);
int64_t ql_lora_wgrad_workspace_floats(int64_t M, int64_t N, int slots);
