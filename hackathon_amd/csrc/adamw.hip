// AdamW over many fp32 parameter tensors in one launch, for gfx950.
//
// The QLoRA step's optimizer updates only the adapters: 2 tensors per adapted projection,
// 196 tensors and 40.4 M fp32 values at the Qwen2.5-7B shape. torch's foreach AdamW spends
// tens of launches on them; this kernel does the whole group in one pass over HBM (read p, g,
// m, v; write p, m, v: 28 B per parameter).
//
// Per element, the operations and their order are those of torch.optim.AdamW (decoupled weight
// decay, bias-corrected moments, non-amsgrad):
//   p  = p * (1 - lr * wd)
//   m  = lerp(m, g, 1 - beta1)            (m + w (g - m) for w < 0.5, else g - (g - m)(1 - w))
//   v  = v * beta2 + (1 - beta2) g g
//   p  = p - step_size * m / (sqrt(v) / sqrt(bias_correction2) + eps)
// with step_size = lr / bias_correction1, the bias corrections 1 - beta^step, and every scalar
// computed by the caller in double (as torch does in Python) and rounded once to fp32.
//
// Work split: the caller's descriptor table (device memory) gives, per tensor, its pointers,
// its length and the index of its first 2048-element chunk; workgroup b finds its tensor by
// binary search over those chunk offsets and updates chunk b - first_chunk of it.
#include "ql_vec.h"

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 2048;  // elements per workgroup

// Every scalar arrives as torch uses it: computed in double by the caller, rounded once to fp32.
struct AdamwScalars {
  float decay;           // 1 - lr * wd
  float beta2, one_minus_beta1, one_minus_beta2;
  float step_size;       // lr / bias_correction1
  float bc2_sqrt;        // sqrt(bias_correction2)
  float eps;
};

QL_DEV void adamw_elem(float& p, float g, float& m, float& v, const AdamwScalars& s) {
  p = p * s.decay;
  const float w = s.one_minus_beta1;
  m = w < 0.5f ? m + w * (g - m) : g - (g - m) * (1.0f - w);
  v = v * s.beta2;
  v = v + s.one_minus_beta2 * g * g;
  const float denom = sqrtf(v) / s.bc2_sqrt + s.eps;
  p = p + (-s.step_size) * (m / denom);
}

__global__ __launch_bounds__(kThreads) void adamw_multi_fp32(const ql_adamw_tensor* __restrict__ table,
                                                             int n_tensors, AdamwScalars s) {
  const int64_t b = blockIdx.x;
  // last tensor whose first chunk is <= b
  int lo = 0, hi = n_tensors - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (table[mid].first_chunk <= b) lo = mid;
    else hi = mid - 1;
  }
  const ql_adamw_tensor t = table[lo];
  const int64_t base = (b - t.first_chunk) * kChunk;
  const int64_t end = base + kChunk < t.numel ? base + kChunk : t.numel;
  const bool vec = ((reinterpret_cast<uintptr_t>(t.param) | reinterpret_cast<uintptr_t>(t.grad) |
                     reinterpret_cast<uintptr_t>(t.exp_avg) |
                     reinterpret_cast<uintptr_t>(t.exp_avg_sq)) & 15) == 0;
  int64_t i = base + 4 * threadIdx.x;
  if (vec) {
    for (; i + 3 < end; i += 4 * kThreads) {
      float4 p = *reinterpret_cast<const float4*>(t.param + i);
      const float4 g = *reinterpret_cast<const float4*>(t.grad + i);
      float4 m = *reinterpret_cast<const float4*>(t.exp_avg + i);
      float4 v = *reinterpret_cast<const float4*>(t.exp_avg_sq + i);
      adamw_elem(p.x, g.x, m.x, v.x, s);
      adamw_elem(p.y, g.y, m.y, v.y, s);
      adamw_elem(p.z, g.z, m.z, v.z, s);
      adamw_elem(p.w, g.w, m.w, v.w, s);
      *reinterpret_cast<float4*>(t.param + i) = p;
      *reinterpret_cast<float4*>(t.exp_avg + i) = m;
      *reinterpret_cast<float4*>(t.exp_avg_sq + i) = v;
    }
  }
  // tail of a vectorised chunk (the few elements past the last full float4), or a whole
  // unaligned chunk, element by element
  const int64_t start = vec ? base + ((end - base) & ~int64_t(3)) : base;
  for (int64_t j = start + threadIdx.x; j < end; j += kThreads) {
    float p = t.param[j], m = t.exp_avg[j], v = t.exp_avg_sq[j];
    adamw_elem(p, t.grad[j], m, v, s);
    t.param[j] = p;
    t.exp_avg[j] = m;
    t.exp_avg_sq[j] = v;
  }
}

}  // namespace

extern "C" int64_t qlora_adamw_chunk_elems(void) { return kChunk; }

extern "C" int qlora_adamw_fp32(const ql_adamw_tensor* table, int n_tensors, int64_t n_chunks,
                                float decay, float beta2, float one_minus_beta1,
                                float one_minus_beta2, float step_size,
                                float bias_correction2_sqrt, float eps, ql_stream_t stream) {
  if (n_tensors < 0 || n_chunks < 0) return QL_EINVAL;
  if (n_tensors == 0 || n_chunks == 0) return QL_OK;
  if (!table || !ql_aligned(table, 8) || n_chunks > INT32_MAX) return QL_EINVAL;
  if (!(bias_correction2_sqrt > 0.f)) return QL_EINVAL;
  AdamwScalars s;
  s.decay = decay;
  s.beta2 = beta2;
  s.one_minus_beta1 = one_minus_beta1;
  s.one_minus_beta2 = one_minus_beta2;
  s.step_size = step_size;
  s.bc2_sqrt = bias_correction2_sqrt;
  s.eps = eps;
  hipLaunchKernelGGL(adamw_multi_fp32, dim3((unsigned)n_chunks), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), table, n_tensors, s);
  return ql_launch_status();
}
