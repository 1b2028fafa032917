// 16-bit matrix transpose, for gfx950: out[c][r] = in[r][c].
//
// Used for operands the NT GEMM wants k-contiguous: the frozen lm_head weight W [V, H]
// becomes W^T [H, V] once (kept while W is unchanged) so that dz @ W of the fused
// cross-entropy (solution/cross_entropy.py:123, solution/fused_ce.py:143) runs as an NT
// GEMM, and the small LoRA matrices are laid out for the rank-16 GEMM segment.
// HBM-bound: one workgroup per 64 x 64 tile, staged through LDS (rows padded by one 32-bit
// word so both the row-wise writes and the column-wise reads spread over the banks); each
// thread moves pairs of 16-bit values so global reads and writes are 4 B per lane and 256 B
// contiguous per 64 lanes.
#include "ql_common.h"

namespace {

constexpr int kTile = 64;
constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void transpose16_kernel(const uint16_t* __restrict__ in,
                                                               int64_t rows, int64_t cols,
                                                               int64_t ld_in,
                                                               uint16_t* __restrict__ out,
                                                               int64_t ld_out) {
  __shared__ uint16_t tile[kTile][kTile + 2];
  const int64_t r0 = (int64_t)blockIdx.y * kTile, c0 = (int64_t)blockIdx.x * kTile;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 column pairs x 8 rows
#pragma unroll
  for (int i = 0; i < kTile / 8; ++i) {
    const int r = ty + 8 * i;
    const int64_t gr = r0 + r, gc = c0 + 2 * tx;
    uint16_t a = 0, b = 0;
    if (gr < rows) {
      if (gc < cols) a = in[gr * ld_in + gc];
      if (gc + 1 < cols) b = in[gr * ld_in + gc + 1];
    }
    tile[r][2 * tx] = a;
    tile[r][2 * tx + 1] = b;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTile / 8; ++i) {
    const int c = ty + 8 * i;  // output row = input column c0 + c
    const int64_t oc = c0 + c, orow = r0 + 2 * tx;
    if (oc < cols) {
      if (orow < rows) out[oc * ld_out + orow] = tile[2 * tx][c];
      if (orow + 1 < rows) out[oc * ld_out + orow + 1] = tile[2 * tx + 1][c];
    }
  }
}

}  // namespace

extern "C" int qlora_transpose16(const void* in, int64_t rows, int64_t cols, int64_t ld_in,
                                 void* out, int64_t ld_out, ql_stream_t stream) {
  if (rows < 0 || cols < 0 || ld_in < cols || ld_out < rows) return QL_EINVAL;
  if (rows == 0 || cols == 0) return QL_OK;
  if (!in || !out) return QL_EINVAL;
  if (!ql_aligned(in, 2) || !ql_aligned(out, 2)) return QL_EALIGN;
  if ((rows + kTile - 1) / kTile > 65535) return QL_EINVAL;
  const dim3 grid((unsigned)((cols + kTile - 1) / kTile), (unsigned)((rows + kTile - 1) / kTile));
  hipLaunchKernelGGL(transpose16_kernel, grid, dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(in), rows,
                     cols, ld_in, static_cast<uint16_t*>(out), ld_out);
  return ql_launch_status();
}
