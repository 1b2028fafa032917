// RMSNorm forward and backward (frozen weight), for gfx950.
//
// Reference semantics: solution/rmsnorm.py:24-39 (forward) and :42-55 (backward):
//   r  = 1 / sqrt(sum(x^2)/N + eps)
//   y  = w * round_{x dtype}(x * r)                 (round only when x is 16-bit)
//   dx = r * (g - x * r^2 * mean(g * x)),  g = dy * w
//
// HBM-bound (per row: fwd reads x once and writes y; bwd reads dy and x and writes dx).
// Fast path: one wavefront per row, 4 rows per 256-thread workgroup. Lane l holds the
// 8-element chunks l, l+64, l+128, ... of its row in registers, so x is read from HBM exactly
// once; each load instruction of the wave covers 64 x 16 B contiguous. The row reduction is
// a 64-lane butterfly (no LDS, no barrier). Fallback (row not a multiple of 8 elements,
// unaligned rows, or rows longer than 8192): one workgroup per row, two passes.
#include "ql_vec.h"

namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;

// ADD: the row is h = round_{x dtype}(x + d) (the residual add of a decoder layer), written
// to `h` and normalised; otherwise the row is x and `d`, `h` are unused.
template <int XT, int WT, int YT, int VPL, bool ADD>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_wave(
    const typename Elem<XT>::T* __restrict__ x, int64_t xs, const typename Elem<XT>::T* __restrict__ d,
    int64_t ds, typename Elem<XT>::T* __restrict__ h, int64_t hs,
    const typename Elem<WT>::T* __restrict__ w, typename Elem<YT>::T* __restrict__ y, int64_t ys,
    float* __restrict__ rstd, int64_t n_rows, int n_cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int nvec = n_cols >> 3;
  const auto* xr = x + row * xs;
  float v[VPL][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = i * 64 + lane;
    if (c < nvec) {
      Vec8<XT>::load(xr + 8 * c, v[i]);
      if constexpr (ADD) {
        float dv[8];
        Vec8<XT>::load(d + row * ds + 8 * c, dv);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[i][j] = round_through<XT>(v[i][j] + dv[j]);
        Vec8<XT>::store(h + row * hs + 8 * c, v[i]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += v[i][j] * v[i][j];
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)n_cols + eps);
  if (lane == 0) rstd[row] = r;
  auto* yr = y + row * ys;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = i * 64 + lane;
    if (c < nvec) {
      float wv[8], o[8];
      Vec8<WT>::load(w + 8 * c, wv);
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = wv[j] * round_through<XT>(v[i][j] * r);
      Vec8<YT>::store(yr + 8 * c, o);
    }
  }
}

// RES: dx also receives the gradient `dres` of the row's other use (the residual stream),
// added in fp32 before the one rounding to dx's dtype.
template <int GT, int XT, int WT, int DXT, int VPL, bool RES>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_wave(
    const typename Elem<GT>::T* __restrict__ dy, int64_t dys, const typename Elem<XT>::T* __restrict__ x,
    int64_t xs, const typename Elem<WT>::T* __restrict__ w, const float* __restrict__ rstd,
    const typename Elem<DXT>::T* __restrict__ dres, int64_t drs,
    typename Elem<DXT>::T* __restrict__ dx, int64_t dxs, int64_t n_rows, int n_cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int nvec = n_cols >> 3;
  float g[VPL][8], xv[VPL][8];
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = i * 64 + lane;
    if (c < nvec) {
      float wv[8];
      Vec8<GT>::load(dy + row * dys + 8 * c, g[i]);
      Vec8<XT>::load(x + row * xs + 8 * c, xv[i]);
      Vec8<WT>::load(w + 8 * c, wv);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        g[i][j] *= wv[j];
        dot += g[i][j] * xv[i][j];
      }
    }
  }
  dot = wave_sum(dot) / (float)n_cols;
  const float r = rstd[row];
  const float k = r * r * dot;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = i * 64 + lane;
    if (c < nvec) {
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = r * (g[i][j] - xv[i][j] * k);
      if constexpr (RES) {
        float rv[8];
        Vec8<DXT>::load(dres + row * drs + 8 * c, rv);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] += rv[j];
      }
      Vec8<DXT>::store(dx + row * dxs + 8 * c, o);
    }
  }
}

// The same backward for long rows (7 or 8 chunks a lane): every load of the row (dy, x, the row's rstd and, for 16-bit rows, dres) goes out before
// the first use, so a wave waits for HBM once per row, and the row stays in registers in its
// loaded (packed) form: the second pass unpacks it again and recomputes g = dy * w with the
// same roundings (contraction off, the fused steps written out: the results are bit-identical
// to keeping g). The weight, the same for every row, is staged once per workgroup in LDS and
// read from there by both passes. A 3584-wide bf16 row then takes 119 registers a lane
// instead of 154: four waves per SIMD,
// so the 4096 rows of a 7B step run in one round instead of 1.33: 32.1 -> 27.8 us with the
// residual gradient, 23.7 -> 21.2 us without, measured on MI355X with inputs cold (rotated
// past the MALL). Short rows (4 chunks) keep rmsnorm_bwd_wave, which has no barrier and was
// faster there (17.4 against 18.2 us at 8192 x 1536).
template <int GT, int XT, int WT, int DXT, int VPL, bool RES>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_wave_packed(
    const typename Elem<GT>::T* __restrict__ dy, int64_t dys, const typename Elem<XT>::T* __restrict__ x,
    int64_t xs, const typename Elem<WT>::T* __restrict__ w, const float* __restrict__ rstd,
    const typename Elem<DXT>::T* __restrict__ dres, int64_t drs,
    typename Elem<DXT>::T* __restrict__ dx, int64_t dxs, int64_t n_rows, int n_cols) {
#pragma clang fp contract(off)
  // dres early only where its packed form saves registers (16-bit) and the row is short
  // enough for it to fit beside dy and x
  constexpr bool kEarlyRes = RES && DXT != QL_F32 && VPL <= 8;
  constexpr int kWBytes = WT == QL_F32 ? 32 : 16;  // one 8-element chunk of w
  __shared__ __attribute__((aligned(16))) char wl[VPL * 64 * kWBytes];
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int nvec = n_cols >> 3;
  for (int c = threadIdx.x; c < nvec; c += kThreads) {  // chunk c of w at wl + c * kWBytes
    Raw8<WT> t;
    t.load(w + 8 * c);
    t.store_bytes(wl + c * kWBytes);
  }
  const bool live = row < n_rows;  // no early return: every wave meets the barrier
  Raw8<GT> gr[VPL];
  Raw8<XT> xr[VPL];
  Raw8<DXT> rr[kEarlyRes ? VPL : 1];
  if (live) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = i * 64 + lane;
      if (c < nvec) {
        gr[i].load(dy + row * dys + 8 * c);
        xr[i].load(x + row * xs + 8 * c);
        if constexpr (kEarlyRes) rr[i].load(dres + row * drs + 8 * c);
      }
    }
  }
  const float r = live ? rstd[row] : 0.f;
  __syncthreads();
  if (!live) return;
  auto weight = [&](int c, float* wv) {
    Raw8<WT> t;
    t.load_bytes(wl + c * kWBytes);
    t.unpack(wv);
  };
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = i * 64 + lane;
    if (c < nvec) {
      float g[8], xv[8], wv[8];
      gr[i].unpack(g);
      xr[i].unpack(xv);
      weight(c, wv);
#pragma unroll
      for (int j = 0; j < 8; ++j) dot = __builtin_fmaf(g[j] * wv[j], xv[j], dot);
    }
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    gr[i].opaque();
    xr[i].opaque();
  }
  dot = wave_sum(dot) / (float)n_cols;
  const float k = r * r * dot;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = i * 64 + lane;
    if (c < nvec) {
      float g[8], xv[8], wv[8], o[8];
      gr[i].unpack(g);
      xr[i].unpack(xv);
      weight(c, wv);
      if constexpr (RES) {  // dx = r (g - x k) + dres, the last step fused
        float rv[8];
        if constexpr (kEarlyRes) rr[i].unpack(rv);
        else Vec8<DXT>::load(dres + row * drs + 8 * c, rv);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          o[j] = __builtin_fmaf(r, __builtin_fmaf(-xv[j], k, g[j] * wv[j]), rv[j]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = r * __builtin_fmaf(-xv[j], k, g[j] * wv[j]);
      }
      Vec8<DXT>::store(dx + row * dxs + 8 * c, o);
    }
  }
}

// ---- fallback: one workgroup per row, any length / alignment, runtime dtypes --------------
QL_DEV float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wid] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) t += red[i];
  __syncthreads();
  return t;
}

__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_generic(
    const void* __restrict__ x, int xt, int64_t xs, const void* __restrict__ w, int wt,
    void* __restrict__ y, int yt, int64_t ys, float* __restrict__ rstd, int n_cols, float eps) {
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  float ss = 0.f;
  for (int c = threadIdx.x; c < n_cols; c += kThreads) {
    const float v = load_any(x, xt, row * xs + c);
    ss += v * v;
  }
  ss = block_sum(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)n_cols + eps);
  if (threadIdx.x == 0) rstd[row] = r;
  for (int c = threadIdx.x; c < n_cols; c += kThreads) {
    const float v = load_any(x, xt, row * xs + c);
    store_any(y, yt, row * ys + c, load_any(w, wt, c) * round_any(v * r, xt));
  }
}

__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_generic(
    const void* __restrict__ dy, int gt, int64_t dys, const void* __restrict__ x, int xt,
    int64_t xs, const void* __restrict__ w, int wt, const float* __restrict__ rstd,
    void* __restrict__ dx, int dxt, int64_t dxs, int n_cols) {
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  float dot = 0.f;
  for (int c = threadIdx.x; c < n_cols; c += kThreads)
    dot += load_any(dy, gt, row * dys + c) * load_any(w, wt, c) * load_any(x, xt, row * xs + c);
  dot = block_sum(dot, red) / (float)n_cols;
  const float r = rstd[row];
  const float k = r * r * dot;
  for (int c = threadIdx.x; c < n_cols; c += kThreads) {
    const float g = load_any(dy, gt, row * dys + c) * load_any(w, wt, c);
    store_any(dx, dxt, row * dxs + c, r * (g - load_any(x, xt, row * xs + c) * k));
  }
}

bool row_vec_ok(const void* p, int64_t stride, int dt) {
  return ql_aligned(p, 16) && ((stride * ql_elem_size(dt)) % 16) == 0;
}

template <int XT, int WT, bool ADD = false>
int fwd_fast(const void* x, int64_t xs, const void* w, void* y, int64_t ys, float* rstd,
             int64_t n_rows, int n_cols, float eps, hipStream_t s, const void* d = nullptr,
             int64_t ds = 0, void* h = nullptr, int64_t hs = 0) {
  constexpr int YT = (XT == WT) ? XT : QL_F32;
  using X = typename Elem<XT>::T;
  using W = typename Elem<WT>::T;
  using Y = typename Elem<YT>::T;
  const dim3 grid((unsigned)((n_rows + kRowsPerBlock - 1) / kRowsPerBlock));
  const int nvec = n_cols / 8;
#define QL_RMS_FWD(VPL)                                                                       \
  hipLaunchKernelGGL((rmsnorm_fwd_wave<XT, WT, YT, VPL, ADD>), grid, dim3(kThreads), 0, s,    \
                     (const X*)x, xs, (const X*)d, ds, (X*)h, hs, (const W*)w, (Y*)y, ys, rstd, \
                     n_rows, n_cols, eps)
  if (nvec <= 4 * 64) QL_RMS_FWD(4);
  else if (nvec <= 8 * 64) QL_RMS_FWD(8);
  else QL_RMS_FWD(16);
#undef QL_RMS_FWD
  return ql_launch_status();
}

template <int XT, int WT, bool RES = false>
int bwd_fast(const void* dy, int64_t dys, const void* x, int64_t xs, const void* w,
             const float* rstd, void* dx, int64_t dxs, int64_t n_rows, int n_cols, hipStream_t s,
             const void* dres = nullptr, int64_t drs = 0) {
  constexpr int GT = (XT == WT) ? XT : QL_F32;  // dy has the forward output's dtype
  using G = typename Elem<GT>::T;
  using X = typename Elem<XT>::T;
  using W = typename Elem<WT>::T;
  const dim3 grid((unsigned)((n_rows + kRowsPerBlock - 1) / kRowsPerBlock));
  const int nvec = n_cols / 8;
#define QL_RMS_BWD(KERNEL, VPL)                                                                 \
  hipLaunchKernelGGL((KERNEL<GT, XT, WT, XT, VPL, RES>), grid, dim3(kThreads), 0, s,             \
                     (const G*)dy, dys, (const X*)x, xs, (const W*)w, rstd, (const X*)dres, drs, \
                     (X*)dx, dxs, n_rows, n_cols)
  if (nvec <= 4 * 64) QL_RMS_BWD(rmsnorm_bwd_wave, 4);
  else if (nvec <= 7 * 64) QL_RMS_BWD(rmsnorm_bwd_wave_packed, 7);  // hidden 3584 (7B): 448 chunks
  else if (nvec <= 8 * 64) QL_RMS_BWD(rmsnorm_bwd_wave_packed, 8);
  else QL_RMS_BWD(rmsnorm_bwd_wave, 16);
#undef QL_RMS_BWD
  return ql_launch_status();
}

}  // namespace

extern "C" int qlora_rmsnorm_fwd(const void* x, int x_dtype, int64_t x_row_stride, const void* w,
                                 int w_dtype, void* y, int y_dtype, int64_t y_row_stride,
                                 float* rstd, int64_t n_rows, int64_t n_cols, float eps,
                                 ql_stream_t stream) {
  if (n_rows < 0 || n_cols <= 0 || n_cols > INT32_MAX) return QL_EINVAL;
  if (!ql_valid_dtype(x_dtype) || !ql_valid_dtype(w_dtype) || !ql_valid_dtype(y_dtype))
    return QL_EDTYPE;
  if (n_rows == 0) return QL_OK;
  if (!x || !w || !y || !rstd) return QL_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nc = (int)n_cols;
  const bool fast = (nc % 8) == 0 && nc <= 16 * 64 * 8 && y_dtype == ql_promote(x_dtype, w_dtype) &&
                    row_vec_ok(x, x_row_stride, x_dtype) && row_vec_ok(y, y_row_stride, y_dtype) &&
                    ql_aligned(w, 16);
  if (fast) {
    QL_DISPATCH_DTYPE2(x_dtype, w_dtype, XT, WT,
                       return fwd_fast<XT, WT>(x, x_row_stride, w, y, y_row_stride, rstd, n_rows,
                                               nc, eps, s));
  }
  hipLaunchKernelGGL(rmsnorm_fwd_generic, dim3((unsigned)n_rows), dim3(kThreads), 0, s, x, x_dtype,
                     x_row_stride, w, w_dtype, y, y_dtype, y_row_stride, rstd, nc, eps);
  return ql_launch_status();
}

extern "C" int qlora_rmsnorm_bwd(const void* dy, int dy_dtype, int64_t dy_row_stride,
                                 const void* x, int x_dtype, int64_t x_row_stride, const void* w,
                                 int w_dtype, const float* rstd, void* dx, int dx_dtype,
                                 int64_t dx_row_stride, int64_t n_rows, int64_t n_cols,
                                 ql_stream_t stream) {
  if (n_rows < 0 || n_cols <= 0 || n_cols > INT32_MAX) return QL_EINVAL;
  if (!ql_valid_dtype(dy_dtype) || !ql_valid_dtype(x_dtype) || !ql_valid_dtype(w_dtype) ||
      !ql_valid_dtype(dx_dtype))
    return QL_EDTYPE;
  if (n_rows == 0) return QL_OK;
  if (!dy || !x || !w || !rstd || !dx) return QL_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nc = (int)n_cols;
  const bool fast = (nc % 8) == 0 && nc <= 16 * 64 * 8 &&
                    dy_dtype == ql_promote(x_dtype, w_dtype) && dx_dtype == x_dtype &&
                    row_vec_ok(dy, dy_row_stride, dy_dtype) && row_vec_ok(x, x_row_stride, x_dtype) &&
                    row_vec_ok(dx, dx_row_stride, dx_dtype) && ql_aligned(w, 16);
  if (fast) {
    QL_DISPATCH_DTYPE2(x_dtype, w_dtype, XT, WT,
                       return bwd_fast<XT, WT>(dy, dy_row_stride, x, x_row_stride, w, rstd, dx,
                                               dx_row_stride, n_rows, nc, s));
  }
  hipLaunchKernelGGL(rmsnorm_bwd_generic, dim3((unsigned)n_rows), dim3(kThreads), 0, s, dy,
                     dy_dtype, dy_row_stride, x, x_dtype, x_row_stride, w, w_dtype, rstd, dx,
                     dx_dtype, dx_row_stride, nc);
  return ql_launch_status();
}

extern "C" int qlora_add_rmsnorm_fwd(const void* x, const void* d, int x_dtype, int64_t x_row_stride,
                                     int64_t d_row_stride, const void* w, int w_dtype, void* h,
                                     int64_t h_row_stride, void* y, int y_dtype,
                                     int64_t y_row_stride, float* rstd, int64_t n_rows,
                                     int64_t n_cols, float eps, ql_stream_t stream) {
  if (n_rows < 0 || n_cols <= 0 || n_cols > INT32_MAX) return QL_EINVAL;
  if (!ql_valid_dtype(x_dtype) || !ql_valid_dtype(w_dtype) || y_dtype != ql_promote(x_dtype, w_dtype))
    return QL_EDTYPE;
  if (n_rows == 0) return QL_OK;
  if (!x || !d || !h || !w || !y || !rstd) return QL_EINVAL;
  const int nc = (int)n_cols;
  if (nc % 8 || nc > 16 * 64 * 8) return QL_ESHAPE;
  if (!row_vec_ok(x, x_row_stride, x_dtype) || !row_vec_ok(d, d_row_stride, x_dtype) ||
      !row_vec_ok(h, h_row_stride, x_dtype) || !row_vec_ok(y, y_row_stride, y_dtype) ||
      !ql_aligned(w, 16))
    return QL_EALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  QL_DISPATCH_DTYPE2(x_dtype, w_dtype, XT, WT,
                     return (fwd_fast<XT, WT, true>(x, x_row_stride, w, y, y_row_stride, rstd,
                                                    n_rows, nc, eps, s, d, d_row_stride, h,
                                                    h_row_stride)));
  return QL_EDTYPE;
}

extern "C" int qlora_rmsnorm_bwd_residual(const void* dy, int dy_dtype, int64_t dy_row_stride,
                                          const void* x, int x_dtype, int64_t x_row_stride,
                                          const void* w, int w_dtype, const float* rstd,
                                          const void* dres, int64_t dres_row_stride, void* dx,
                                          int64_t dx_row_stride, int64_t n_rows, int64_t n_cols,
                                          ql_stream_t stream) {
  if (n_rows < 0 || n_cols <= 0 || n_cols > INT32_MAX) return QL_EINVAL;
  if (!ql_valid_dtype(x_dtype) || !ql_valid_dtype(w_dtype) || dy_dtype != ql_promote(x_dtype, w_dtype))
    return QL_EDTYPE;
  if (n_rows == 0) return QL_OK;
  if (!dy || !x || !w || !rstd || !dres || !dx) return QL_EINVAL;
  const int nc = (int)n_cols;
  if (nc % 8 || nc > 16 * 64 * 8) return QL_ESHAPE;
  if (!row_vec_ok(dy, dy_row_stride, dy_dtype) || !row_vec_ok(x, x_row_stride, x_dtype) ||
      !row_vec_ok(dres, dres_row_stride, x_dtype) || !row_vec_ok(dx, dx_row_stride, x_dtype) ||
      !ql_aligned(w, 16))
    return QL_EALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  QL_DISPATCH_DTYPE2(x_dtype, w_dtype, XT, WT,
                     return (bwd_fast<XT, WT, true>(dy, dy_row_stride, x, x_row_stride, w, rstd, dx,
                                                    dx_row_stride, n_rows, nc, s, dres,
                                                    dres_row_stride)));
  return QL_EDTYPE;
}
