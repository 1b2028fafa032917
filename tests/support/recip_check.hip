// Exhaustive device check of the SwiGLU kernels' fp32 sigmoid (hackathon_amd/csrc/ql_swiglu.h):
//   mode 0: for every fp32 bit pattern d in [lo, hi), ql_recip_fast(d) against 1.0f / d (the
//           correctly rounded division hipcc emits);
//   mode 1: for every fp32 bit pattern x in [lo, hi), against 1.0f / (1.0f + __expf(-x)):
//           ql_sigmoid(x), ql_sigmoid_as<true>(x) wherever ql_sigmoid_fast_ok holds (for x
//           alone or for the eight consecutive patterns it is tested with), and the
//           eight-wide forward ql_swiglu_fwd8(x, 1); two NaNs count as equal.
// Test support only (tests/test_gpu_sigmoid_recip.py); not part of the library.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "../../hackathon_amd/csrc/ql_swiglu.h"

namespace {

__device__ __noinline__ float div_reference(float d) { return 1.0f / d; }

__device__ bool same(float a, float b) {
  return __float_as_uint(a) == __float_as_uint(b) || (a != a && b != b);
}

constexpr uint32_t kPer = 64;  // patterns per thread (a multiple of 8)

__global__ __launch_bounds__(256) void check_kernel(int mode, uint64_t lo, uint64_t hi,
                                                    uint32_t* count, uint32_t* first) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t b0 = lo + t * kPer;
  uint32_t n = 0, f = 0xffffffffu;
  const float ones[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
  for (uint32_t i = 0; i < kPer; i += 8) {
    float v[8], got[8], want[8];
    bool in[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint64_t b = b0 + i + e;
      in[e] = b < hi;
      v[e] = __uint_as_float((uint32_t)(in[e] ? b : lo));
    }
    if (mode == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        got[e] = ql_recip_fast(v[e]);
        want[e] = div_reference(v[e]);
      }
    } else {
      const bool ok8 = ql_sigmoid_fast_ok8(v);
      float x8[8];
      ql_swiglu_fwd8(v, ones, x8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        want[e] = div_reference(1.0f + __expf(-v[e]));
        // the kernels' three forms: the guarded scalar, the fast form wherever its guard
        // holds, and the eight-wide forward (x * sigmoid(x) * 1, against x * want * 1)
        const float s1 = ql_sigmoid(v[e]);
        const float sf = ok8 || ql_sigmoid_fast_ok(v[e]) ? ql_sigmoid_as<true>(v[e]) : want[e];
        const float f8 = v[e] * want[e] * 1.0f;
        got[e] = !same(s1, want[e]) ? s1 : !same(sf, want[e]) ? sf : !same(x8[e], f8) ? NAN : want[e];
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (in[e] && !same(got[e], want[e])) {
        if (n == 0) f = __float_as_uint(v[e]);
        ++n;
      }
  }
  count[t] = n;
  first[t] = f;
}

}  // namespace

// Patterns in [lo, hi) (hi <= 2^32) that differ; *first_bad = the smallest such pattern, or
// 0xffffffff. Returns 0, or a HIP error code.
extern "C" int recip_check(int mode, uint64_t lo, uint64_t hi, uint64_t* mismatches,
                           uint32_t* first_bad) {
  constexpr uint32_t kBlocks = 16384, kThreads = 256;
  constexpr uint64_t kSpan = (uint64_t)kBlocks * kThreads * kPer;  // 2^28 patterns per launch
  const size_t n = (size_t)kBlocks * kThreads;
  uint32_t *dc = nullptr, *df = nullptr;
  hipError_t e = hipMalloc(&dc, n * 4);
  if (e == hipSuccess) e = hipMalloc(&df, n * 4);
  uint32_t* hc = static_cast<uint32_t*>(malloc(n * 4));
  uint32_t* hf = static_cast<uint32_t*>(malloc(n * 4));
  uint64_t bad = 0;
  uint32_t fb = 0xffffffffu;
  for (uint64_t s = lo; e == hipSuccess && s < hi; s += kSpan) {
    hipLaunchKernelGGL(check_kernel, dim3(kBlocks), dim3(kThreads), 0, 0, mode, s,
                       s + kSpan < hi ? s + kSpan : hi, dc, df);
    e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(hc, dc, n * 4, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(hf, df, n * 4, hipMemcpyDeviceToHost);
    for (size_t i = 0; e == hipSuccess && i < n; ++i) {
      bad += hc[i];
      if (hc[i] && hf[i] < fb) fb = hf[i];
    }
  }
  free(hc);
  free(hf);
  if (dc) (void)hipFree(dc);
  if (df) (void)hipFree(df);
  *mismatches = bad;
  *first_bad = fb;
  return (int)e;
}
