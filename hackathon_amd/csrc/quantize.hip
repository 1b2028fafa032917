// NF4 quantisation with a double-quantised absmax, for gfx950: the format producer that
// feeds the dequant kernel (the weight format of solution/nf4.py:73-86, which the reference
// takes from bitsandbytes' quantize_4bit; this kernel produces the same layout without it).
//
//   stage 1  per NF4 block of `blocksize` weights (the lanes of a wave sharing each block when
//            blocksize is a power of two from 16 to 512, else one thread a block): absmax = max |w|, codes =
//            nearest NF4 level of w * (1 / absmax) (fp32 multiply by the correctly rounded
//            reciprocal; ties go to the lower level, i.e. the count of level midpoints
//            strictly below the value), two codes per byte, high nibble first.
//   stage 2  (double quantisation) offset = mean(absmax), accumulated in fp64: for the block
//            absmax of a weight tensor the fp64 sum is exact, so the offset does not depend on
//            the reduction order, and is rounded once to fp32.
//   stage 3  one workgroup per 256 absmax values: absmax2 = max |absmax - offset|, codes =
//            nearest entry of the 256-level dynamic map of (absmax - offset) / absmax2.
// Every step uses the same fp32 operations, in the same order, as the torch quantizer in
// hackathon_amd/quant.py, so the two produce identical bytes.
#include "ql_vec.h"

namespace {

constexpr int kThreads = 256;

// Number of the n sorted midpoints strictly below x (lower bound).
QL_DEV int count_below(const float* mids, int n, float x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (mids[mid] < x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

template <int IT>
__global__ __launch_bounds__(kThreads) void nf4_quantize_blocks(
    const typename Elem<IT>::T* __restrict__ w, int64_t n, int64_t blocksize, int64_t n_blocks,
    const float* __restrict__ nf4_code, uint8_t* __restrict__ packed, float* __restrict__ absmax) {
#pragma clang fp contract(off)
  __shared__ float mids[15];
  if (threadIdx.x < 15) mids[threadIdx.x] = (nf4_code[threadIdx.x] + nf4_code[threadIdx.x + 1]) * 0.5f;
  __syncthreads();
  const int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (b >= n_blocks) return;
  const int64_t j0 = b * blocksize;
  const int64_t j1 = j0 + blocksize < n ? j0 + blocksize : n;
  float am = 0.f;
  for (int64_t j = j0; j < j1; ++j) am = fmaxf(am, fabsf(Elem<IT>::load(w, j)));
  const float inv = am > 0.f ? 1.0f / am : 0.f;
  for (int64_t j = j0; j < j1; j += 2) {  // j0 and n are even
    const int hi = count_below(mids, 15, Elem<IT>::load(w, j) * inv);
    const int lo = count_below(mids, 15, Elem<IT>::load(w, j + 1) * inv);
    packed[j / 2] = (uint8_t)((hi << 4) | lo);
  }
  absmax[b] = am;
}

// Stage 1 with the lanes of a wave sharing the blocks (blocksize = 8 LPB, a power of two from
// 16 to 512): lane l takes the 8 consecutive weights of group g0 + l (one 16-B load of 16-bit
// weights, so a wave's load instruction reads 1 KiB contiguous), the LPB lanes of a block
// combine their maxima with butterflies, and each lane writes its 8 codes as one 32-bit word.
// The per-weight arithmetic is nf4_quantize_blocks': the same absmax, reciprocal and product,
// and the same count of midpoints strictly below the product v, found by table: the 256
// buckets [i / 128 - 1, (i + 1) / 128 - 1) each hold at most one midpoint (the midpoints are
// more than 1/128 apart), so the count is the number of midpoints below the bucket plus
// whether the bucket's own midpoint is below v. The bucket is floor(128 v), exact in fp32,
// clamped to the table (|v| exceeds 1 by at most rounding; NaN goes to bucket 0 and count 0,
// as in the binary search), so the bytes are identical; the GPU tests check them at every
// bucket edge and midpoint and one ulp either side.
static_assert(kThreads == 256, "nf4_quantize_lanes builds its 256-bucket table one bucket a thread");

template <int IT, int LPB>
__global__ __launch_bounds__(kThreads) void nf4_quantize_lanes(
    const typename Elem<IT>::T* __restrict__ w, int64_t n, int64_t n_blocks,
    const float* __restrict__ nf4_code, uint8_t* __restrict__ packed, float* __restrict__ absmax) {
#pragma clang fp contract(off)
  __shared__ float2 lut[256];  // {the bucket's midpoint or +inf, midpoints below the bucket}
  {
    float mid[15];
#pragma unroll
    for (int k = 0; k < 15; ++k) mid[k] = (nf4_code[k] + nf4_code[k + 1]) * 0.5f;
    const int t = threadIdx.x;  // kThreads == 256: one bucket a thread
    const float lo = (float)t / 128.f - 1.f, hi = (float)(t + 1) / 128.f - 1.f;
    float below = 0.f, m = INFINITY;
#pragma unroll
    for (int k = 0; k < 15; ++k) {
      below += mid[k] < lo ? 1.f : 0.f;
      if (mid[k] >= lo && mid[k] < hi) m = mid[k];
    }
    lut[t] = make_float2(m, below);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t n_waves = (int64_t)gridDim.x * (kThreads / 64);
  const int64_t n_groups = (n + 7) / 8;
  // two 64-group spans a step, both loaded before either is coded
  for (int64_t g0 = wave * 128; g0 < n_groups; g0 += n_waves * 128) {  // wave-uniform bounds
    float xs[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t j0 = 8 * (g0 + 64 * u + lane);
      if (j0 + 8 <= n) {
        Vec8<IT>::load(w + j0, xs[u]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xs[u][e] = j0 + e < n ? Elem<IT>::load(w, j0 + e) : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t grp = g0 + 64 * u + lane;
      const int64_t j0 = 8 * grp;
      const bool whole = j0 + 8 <= n;
      const float* x = xs[u];
      float am = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(x[e]));
#pragma unroll
      for (int off = 1; off < LPB; off <<= 1) am = fmaxf(am, __shfl_xor(am, off, 64));
      const float inv = am > 0.f ? 1.0f / am : 0.f;
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = x[e] * inv;
        const float f = fminf(fmaxf(floorf(v * 128.f), -128.f), 127.f);
        const float2 b = lut[(int)f + 128];
        const uint32_t c = (uint32_t)b.y + (b.x < v ? 1u : 0u);
        word |= c << (8 * (e >> 1) + ((e & 1) ? 0 : 4));  // weight 2i: high nibble of byte i
      }
      if (whole) {
        *reinterpret_cast<uint32_t*>(packed + 4 * grp) = word;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (j0 + 2 * i < n) packed[4 * grp + i] = (uint8_t)(word >> (8 * i));
      }
      const int64_t blk = grp / LPB;
      if (lane % LPB == 0 && blk < n_blocks) absmax[blk] = am;
    }
  }
}

// fp64 partial sums of x[0..n): one per workgroup.
__global__ __launch_bounds__(kThreads) void sum_f64_partials(const float* __restrict__ x,
                                                             int64_t n, double* __restrict__ part) {
  __shared__ double red[kThreads / 64];
  double s = 0.0;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    s += (double)x[i];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

// offset = (float)(sum(part) / n), one wave (the fp64 sum is exact, so in any order).
__global__ __launch_bounds__(64) void mean_from_partials(const double* __restrict__ part,
                                                         int n_part, int64_t n,
                                                         float* __restrict__ offset) {
  double s = 0.0;
  for (int i = threadIdx.x; i < n_part; i += 64) s += part[i];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if (threadIdx.x == 0) offset[0] = (float)(s / (double)n);
}

// One workgroup per block of 256 values of (absmax - offset): dynamic-map codes + absmax2.
__global__ __launch_bounds__(kThreads) void quantize8_blocks(
    const float* __restrict__ absmax, int64_t n, const float* __restrict__ offset,
    const float* __restrict__ code2, uint8_t* __restrict__ codes, float* __restrict__ absmax2) {
#pragma clang fp contract(off)
  __shared__ float mids[255];
  __shared__ float red[kThreads / 64];
  if (threadIdx.x < 255) mids[threadIdx.x] = (code2[threadIdx.x] + code2[threadIdx.x + 1]) * 0.5f;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const float v = i < n ? absmax[i] - offset[0] : 0.f;
  float m = fabsf(v);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  const float am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float inv = am > 0.f ? 1.0f / am : 0.f;
  if (i < n) codes[i] = (uint8_t)count_below(mids, 255, v * inv);
  if (threadIdx.x == 0) absmax2[blockIdx.x] = am;
}

constexpr int kPartials = 256;

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

}  // namespace

extern "C" int64_t qlora_nf4_quantize_workspace_size(int64_t n, int blocksize, int nested) {
  if (n <= 0 || blocksize <= 0 || !nested) return 0;
  const int64_t nb = (n + blocksize - 1) / blocksize;
  return align256(nb * (int64_t)sizeof(float)) + kPartials * (int64_t)sizeof(double);
}

extern "C" int qlora_nf4_quantize(const void* w, int w_dtype, int64_t n, int blocksize, int nested,
                                  int blocksize2, const float* nf4_code, const float* code2,
                                  uint8_t* packed, void* absmax, float* absmax2, float* offset,
                                  void* workspace, int64_t workspace_bytes, ql_stream_t stream) {
  if (n < 0 || (n & 1) || blocksize < 2 || (blocksize & 1)) return QL_EINVAL;
  if (nested && blocksize2 != 256) return QL_EINVAL;  // one workgroup per 256-value block
  if (n == 0) return QL_OK;
  if (!w || !nf4_code || !packed || !absmax) return QL_EINVAL;
  if (nested && (!code2 || !absmax2 || !offset)) return QL_EINVAL;
  if (!ql_valid_dtype(w_dtype)) return QL_EDTYPE;
  const int64_t nb = (n + blocksize - 1) / blocksize;
  if (nested && (workspace_bytes < qlora_nf4_quantize_workspace_size(n, blocksize, nested) ||
                 !workspace || !ql_aligned(workspace, 16)))
    return QL_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* am = nested ? static_cast<float*>(workspace) : static_cast<float*>(absmax);
  const int lpb = blocksize / 8;
  const bool lanes = (blocksize & (blocksize - 1)) == 0 && blocksize >= 16 && blocksize <= 512 &&
                     ql_aligned(w, 16) && ql_aligned(packed, 4);
  if (lanes) {
    const int64_t waves = (n / 8 + 128) / 128;
    const int64_t wgs = (waves + kThreads / 64 - 1) / (kThreads / 64);
    const dim3 g1((unsigned)(wgs < 65536 ? wgs : 65536));
#define QL_QZ(LPB)                                                                               \
  QL_DISPATCH_DTYPE(w_dtype, DT,                                                                 \
                    hipLaunchKernelGGL((nf4_quantize_lanes<DT, LPB>), g1, dim3(kThreads), 0, s,  \
                                       static_cast<const typename Elem<DT>::T*>(w), n, nb,       \
                                       nf4_code, packed, am))
    switch (lpb) {
      case 2: QL_QZ(2); break;
      case 4: QL_QZ(4); break;
      case 8: QL_QZ(8); break;
      case 16: QL_QZ(16); break;
      case 32: QL_QZ(32); break;
      default: QL_QZ(64); break;
    }
#undef QL_QZ
  } else {
    const dim3 g1((unsigned)((nb + kThreads - 1) / kThreads));
    QL_DISPATCH_DTYPE(w_dtype, DT,
                      hipLaunchKernelGGL((nf4_quantize_blocks<DT>), g1, dim3(kThreads), 0, s,
                                         static_cast<const typename Elem<DT>::T*>(w), n,
                                         (int64_t)blocksize, nb, nf4_code, packed, am));
  }
  if (!nested) return ql_launch_status();
  double* part = reinterpret_cast<double*>(static_cast<char*>(workspace) +
                                           align256(nb * (int64_t)sizeof(float)));
  hipLaunchKernelGGL(sum_f64_partials, dim3(kPartials), dim3(kThreads), 0, s, am, nb, part);
  hipLaunchKernelGGL(mean_from_partials, dim3(1), dim3(64), 0, s, part, kPartials, nb, offset);
  const dim3 g3((unsigned)((nb + 255) / 256));
  hipLaunchKernelGGL(quantize8_blocks, g3, dim3(kThreads), 0, s, am, nb, offset, code2,
                     static_cast<uint8_t*>(absmax), absmax2);
  return ql_launch_status();
}
