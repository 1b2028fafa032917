// Per-row cross-entropy statistics over a chunk of logits, with the in-place gradient,
// for gfx950.
//
// Reference semantics: solution/fused_ce.py:42-96 (ce_row_kernel) and
// solution/cross_entropy.py:48-90 (fused_ce_kernel). Per row z[0..V):
//   m = max z, s = sum exp(z - m), t = sum exp(z - m) * z
//   lse = m + log s ; entropy = lse - t / s ; argmax = first index of the maximum
//   loss = labelled ? lse - z[target] : 0
//   dz   = (exp(z - lse) - [v == target]) * (labelled ? grad_scale : 0)   (in place)
//
// HBM-bound: sweep 1 reads the row, sweep 2 reads it again and overwrites it with dz.
// One 512-thread workgroup per row; each thread walks 8-element (16 B) chunks with a stride
// of the workgroup, keeping a running (m, s, t, best, best_idx) per thread, rescaling once
// per chunk. Threads combine through wave butterflies and one LDS exchange.
#include "ql_vec.h"

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr float kLog2e = 1.4426950408889634f;

struct RowStat {
  float m, s, t, best;
  int64_t best_idx;
};

QL_DEV void merge(RowStat& a, const RowStat& b) {
  // (m, s, t): rescale both sides to the larger max. best: larger value, then lower index.
  const float m = fmaxf(a.m, b.m);
  const float fa = (a.m == -INFINITY) ? 0.f : exp2f((a.m - m) * kLog2e);
  const float fb = (b.m == -INFINITY) ? 0.f : exp2f((b.m - m) * kLog2e);
  a.s = a.s * fa + b.s * fb;
  a.t = a.t * fa + b.t * fb;
  a.m = m;
  if (b.best > a.best || (b.best == a.best && b.best_idx < a.best_idx)) {
    a.best = b.best;
    a.best_idx = b.best_idx;
  }
}

QL_DEV RowStat shfl_stat(const RowStat& v, int off) {
  RowStat r;
  r.m = __shfl_xor(v.m, off, 64);
  r.s = __shfl_xor(v.s, off, 64);
  r.t = __shfl_xor(v.t, off, 64);
  r.best = __shfl_xor(v.best, off, 64);
  r.best_idx = __shfl_xor(v.best_idx, off, 64);
  return r;
}

template <int DT, int VW>
__global__ __launch_bounds__(kThreads) void ce_rows_kernel(
    typename Elem<DT>::T* __restrict__ logits, int64_t row_stride, int64_t V,
    const int64_t* __restrict__ target, float* __restrict__ loss, float* __restrict__ entropy,
    int32_t* __restrict__ correct, int64_t* __restrict__ pred, int ignore_mode, int write_grad,
    float grad_scale) {
  __shared__ RowStat part[kWaves];
  __shared__ float lse_sh;
  const int64_t row = blockIdx.x;
  auto* z = logits + row * row_stride;
  const int64_t tgt = target[row];
  const bool labelled = ignore_mode == 0 ? (tgt >= 0) : (tgt != -100);

  RowStat st{-INFINITY, 0.f, 0.f, -INFINITY, 0};
  const int64_t nchunk = V / VW;
  for (int64_t c = threadIdx.x; c < nchunk; c += kThreads) {
    float v[VW];
    if constexpr (VW == 8) Vec8<DT>::load(z + 8 * c, v);
    else v[0] = Elem<DT>::to_f32(z[c]);
    float cm = v[0];
    int cj = 0;
#pragma unroll
    for (int j = 1; j < VW; ++j)
      if (v[j] > cm) { cm = v[j]; cj = j; }
    if (cm > st.best) { st.best = cm; st.best_idx = c * VW + cj; }
    const float m = fmaxf(st.m, cm);
    const float alpha = (st.m == -INFINITY) ? 0.f : exp2f((st.m - m) * kLog2e);
    float es = 0.f, et = 0.f;
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float e = exp2f((v[j] - m) * kLog2e);
      es += e;
      et += e * v[j];
    }
    st.s = st.s * alpha + es;
    st.t = st.t * alpha + et;
    st.m = m;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) merge(st, shfl_stat(st, off));
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) part[wid] = st;
  __syncthreads();
  if (threadIdx.x == 0) {
    RowStat a = part[0];
    for (int i = 1; i < kWaves; ++i) merge(a, part[i]);
    const float lse = a.m + logf(a.s);
    lse_sh = lse;
    // A label outside [0, V) is never read (the loss becomes NaN instead of a stray load).
    const bool in_range = tgt >= 0 && tgt < V;
    const float zt = (labelled && in_range) ? Elem<DT>::to_f32(z[tgt]) : NAN;
    loss[row] = labelled ? lse - zt : 0.f;
    entropy[row] = lse - a.t / a.s;
    if (correct) correct[row] = (labelled && a.best_idx == tgt) ? 1 : 0;
    if (pred) pred[row] = a.best_idx;
  }
  if (!write_grad) return;
  __syncthreads();
  const float lse = lse_sh;
  const float gs = labelled ? grad_scale : 0.f;
  for (int64_t c = threadIdx.x; c < nchunk; c += kThreads) {
    float v[VW];
    if constexpr (VW == 8) Vec8<DT>::load(z + 8 * c, v);
    else v[0] = Elem<DT>::to_f32(z[c]);
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float onehot = (c * VW + j == tgt) ? 1.f : 0.f;
      v[j] = (exp2f((v[j] - lse) * kLog2e) - onehot) * gs;
    }
    if constexpr (VW == 8) Vec8<DT>::store(z + 8 * c, v);
    else z[c] = Elem<DT>::from_f32(v[0]);
  }
}

template <int DT>
int launch_ce(void* logits, int64_t rs, int64_t n_rows, int64_t V, const int64_t* target,
              float* loss, float* entropy, int32_t* correct, int64_t* pred, int ignore_mode,
              int write_grad, float grad_scale, hipStream_t s) {
  using T = typename Elem<DT>::T;
  const bool vec = (V % 8) == 0 && ql_aligned(logits, 16) && ((rs * ql_elem_size(DT)) % 16) == 0;
  if (vec)
    hipLaunchKernelGGL((ce_rows_kernel<DT, 8>), dim3((unsigned)n_rows), dim3(kThreads), 0, s,
                       (T*)logits, rs, V, target, loss, entropy, correct, pred, ignore_mode,
                       write_grad, grad_scale);
  else
    hipLaunchKernelGGL((ce_rows_kernel<DT, 1>), dim3((unsigned)n_rows), dim3(kThreads), 0, s,
                       (T*)logits, rs, V, target, loss, entropy, correct, pred, ignore_mode,
                       write_grad, grad_scale);
  return ql_launch_status();
}

}  // namespace

extern "C" int qlora_ce_rows(void* logits, int logits_dtype, int64_t row_stride, int64_t n_rows,
                             int64_t vocab, const int64_t* target, float* loss, float* entropy,
                             int32_t* correct, int64_t* pred, int ignore_mode, int write_grad,
                             float grad_scale, ql_stream_t stream) {
  if (n_rows < 0 || vocab <= 0 || n_rows > UINT32_MAX) return QL_EINVAL;
  if (ignore_mode != 0 && ignore_mode != 1) return QL_EINVAL;
  if (!ql_valid_dtype(logits_dtype)) return QL_EDTYPE;
  if (n_rows == 0) return QL_OK;
  if (!logits || !target || !loss || !entropy) return QL_EINVAL;
  QL_DISPATCH_DTYPE(logits_dtype, DT,
                    return launch_ce<DT>(logits, row_stride, n_rows, vocab, target, loss, entropy,
                                         correct, pred, ignore_mode, write_grad, grad_scale,
                                         static_cast<hipStream_t>(stream)));
  return QL_EDTYPE;
}
