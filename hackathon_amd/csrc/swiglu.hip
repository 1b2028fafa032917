// SwiGLU forward/backward, for gfx950.
//
// Reference semantics: solution/swiglu.py:15-22 and :25-37, all math in fp32:
//   out   = gate * sigmoid(gate) * up
//   dup   = g * gate * sig
//   dgate = g * up * sig * (1 + gate * (1 - sig))
//
// HBM-bound: fwd 2 reads + 1 write, bwd 3 reads + 2 writes per element. Each thread handles
// 8 consecutive elements per step (16 B per tensor for 16-bit dtypes) in a grid-stride loop
// sized to a few waves per SIMD, so each wave-level access is 1 KiB contiguous.
#include "ql_swiglu.h"
#include "ql_vec.h"

namespace {

constexpr int kThreads = 256;

template <int DT>
__global__ __launch_bounds__(kThreads) void swiglu_fwd_vec(const typename Elem<DT>::T* __restrict__ gate,
                                                           const typename Elem<DT>::T* __restrict__ up,
                                                           typename Elem<DT>::T* __restrict__ out,
                                                           int64_t n_vec) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n_vec;
       i += (int64_t)gridDim.x * kThreads) {
    float g[8], u[8], o[8];
    Vec8<DT>::load(gate + 8 * i, g);
    Vec8<DT>::load(up + 8 * i, u);
    ql_swiglu_fwd8(g, u, o);
    Vec8<DT>::store(out + 8 * i, o);
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_vec(
    const typename Elem<DT>::T* __restrict__ grad, const typename Elem<DT>::T* __restrict__ gate,
    const typename Elem<DT>::T* __restrict__ up, typename Elem<DT>::T* __restrict__ dgate,
    typename Elem<DT>::T* __restrict__ dup, int64_t n_vec) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n_vec;
       i += (int64_t)gridDim.x * kThreads) {
    float gr[8], g[8], u[8], dg[8], du[8];
    Vec8<DT>::load(grad + 8 * i, gr);
    Vec8<DT>::load(gate + 8 * i, g);
    Vec8<DT>::load(up + 8 * i, u);
    ql_swiglu_bwd8(gr, g, u, dg, du);
    Vec8<DT>::store(dgate + 8 * i, dg);
    Vec8<DT>::store(dup + 8 * i, du);
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void swiglu_fwd_scalar(const typename Elem<DT>::T* __restrict__ gate,
                                                              const typename Elem<DT>::T* __restrict__ up,
                                                              typename Elem<DT>::T* __restrict__ out,
                                                              int64_t begin, int64_t n) {
  const int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  Elem<DT>::store(out, i, ql_swiglu_fwd1(Elem<DT>::load(gate, i), Elem<DT>::load(up, i)));
}

template <int DT>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_scalar(
    const typename Elem<DT>::T* __restrict__ grad, const typename Elem<DT>::T* __restrict__ gate,
    const typename Elem<DT>::T* __restrict__ up, typename Elem<DT>::T* __restrict__ dgate,
    typename Elem<DT>::T* __restrict__ dup, int64_t begin, int64_t n) {
  const int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  float dg, du;
  ql_swiglu_bwd1(Elem<DT>::load(grad, i), Elem<DT>::load(gate, i), Elem<DT>::load(up, i), dg, du);
  Elem<DT>::store(dup, i, du);
  Elem<DT>::store(dgate, i, dg);
}

// Row-strided forms for gate / up (and their gradients) that are column ranges of wider
// buffers, e.g. the two halves of one fused gate|up projection output. A grid-stride loop
// over the rows x cols/8 vectors of 8 elements (16 B per tensor); cols, leading dimensions and
// pointers are 16-B granular (checked by the host).
template <int DT>
__global__ __launch_bounds__(kThreads) void swiglu_fwd_rows(
    const typename Elem<DT>::T* __restrict__ gate, int64_t ldg,
    const typename Elem<DT>::T* __restrict__ up, int64_t ldu, typename Elem<DT>::T* __restrict__ out,
    int64_t ldo, int64_t cv, int64_t n_vec) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n_vec;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / cv, c = 8 * (i - r * cv);
    float g[8], u[8], o[8];
    Vec8<DT>::load(gate + r * ldg + c, g);
    Vec8<DT>::load(up + r * ldu + c, u);
    ql_swiglu_fwd8(g, u, o);
    Vec8<DT>::store(out + r * ldo + c, o);
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void swiglu_bwd_rows(
    const typename Elem<DT>::T* __restrict__ grad, int64_t ldgr,
    const typename Elem<DT>::T* __restrict__ gate, int64_t ldg,
    const typename Elem<DT>::T* __restrict__ up, int64_t ldu,
    typename Elem<DT>::T* __restrict__ dgate, int64_t lddg, typename Elem<DT>::T* __restrict__ dup,
    int64_t lddu, int64_t cv, int64_t n_vec) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n_vec;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / cv, c = 8 * (i - r * cv);
    float gr[8], g[8], u[8], dg[8], du[8];
    Vec8<DT>::load(grad + r * ldgr + c, gr);
    Vec8<DT>::load(gate + r * ldg + c, g);
    Vec8<DT>::load(up + r * ldu + c, u);
    ql_swiglu_bwd8(gr, g, u, dg, du);
    Vec8<DT>::store(dgate + r * lddg + c, dg);
    Vec8<DT>::store(dup + r * lddu + c, du);
  }
}

unsigned stream_grid(int64_t n_vec) {
  // 256 CUs x 8 workgroups of 4 waves keeps enough 16-byte accesses in flight for HBM.
  const int64_t cap = 256 * 8;
  const int64_t need = (n_vec + kThreads - 1) / kThreads;
  return (unsigned)(need < cap ? (need > 0 ? need : 1) : cap);
}

template <int DT>
int fwd(const void* gate, const void* up, void* out, int64_t n, hipStream_t s) {
  using T = typename Elem<DT>::T;
  const bool vec = ql_aligned(gate, 16) && ql_aligned(up, 16) && ql_aligned(out, 16);
  int64_t done = 0;
  if (vec && n >= 8) {
    const int64_t nv = n / 8;
    hipLaunchKernelGGL((swiglu_fwd_vec<DT>), dim3(stream_grid(nv)), dim3(kThreads), 0, s,
                       (const T*)gate, (const T*)up, (T*)out, nv);
    done = nv * 8;
  }
  if (done < n)
    hipLaunchKernelGGL((swiglu_fwd_scalar<DT>), dim3((unsigned)((n - done + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, (const T*)gate, (const T*)up, (T*)out, done, n);
  return ql_launch_status();
}

template <int DT>
int bwd(const void* grad, const void* gate, const void* up, void* dgate, void* dup, int64_t n,
        hipStream_t s) {
  using T = typename Elem<DT>::T;
  const bool vec = ql_aligned(grad, 16) && ql_aligned(gate, 16) && ql_aligned(up, 16) &&
                   ql_aligned(dgate, 16) && ql_aligned(dup, 16);
  int64_t done = 0;
  if (vec && n >= 8) {
    const int64_t nv = n / 8;
    hipLaunchKernelGGL((swiglu_bwd_vec<DT>), dim3(stream_grid(nv)), dim3(kThreads), 0, s,
                       (const T*)grad, (const T*)gate, (const T*)up, (T*)dgate, (T*)dup, nv);
    done = nv * 8;
  }
  if (done < n)
    hipLaunchKernelGGL((swiglu_bwd_scalar<DT>), dim3((unsigned)((n - done + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, (const T*)grad, (const T*)gate, (const T*)up,
                       (T*)dgate, (T*)dup, done, n);
  return ql_launch_status();
}

}  // namespace

extern "C" int qlora_swiglu_fwd(const void* gate, const void* up, void* out, int dtype, int64_t n,
                                ql_stream_t stream) {
  if (n < 0) return QL_EINVAL;
  if (!ql_valid_dtype(dtype)) return QL_EDTYPE;
  if (n == 0) return QL_OK;
  if (!gate || !up || !out) return QL_EINVAL;
  QL_DISPATCH_DTYPE(dtype, DT, return fwd<DT>(gate, up, out, n, static_cast<hipStream_t>(stream)));
  return QL_EDTYPE;
}

extern "C" int qlora_swiglu_bwd(const void* grad, const void* gate, const void* up, void* dgate,
                                void* dup, int dtype, int64_t n, ql_stream_t stream) {
  if (n < 0) return QL_EINVAL;
  if (!ql_valid_dtype(dtype)) return QL_EDTYPE;
  if (n == 0) return QL_OK;
  if (!grad || !gate || !up || !dgate || !dup) return QL_EINVAL;
  QL_DISPATCH_DTYPE(dtype, DT,
                    return bwd<DT>(grad, gate, up, dgate, dup, n, static_cast<hipStream_t>(stream)));
  return QL_EDTYPE;
}

namespace {
bool rows_ok(const void* p, int64_t ld, int dtype) {
  return ql_aligned(p, 16) && (ld * ql_elem_size(dtype)) % 16 == 0;
}
}  // namespace

extern "C" int qlora_swiglu_fwd_rows(const void* gate, int64_t ldg, const void* up, int64_t ldu,
                                     void* out, int64_t ldo, int64_t rows, int64_t cols,
                                     int dtype, ql_stream_t stream) {
  if (rows < 0 || cols < 0) return QL_EINVAL;
  if (!ql_valid_dtype(dtype)) return QL_EDTYPE;
  if (rows == 0 || cols == 0) return QL_OK;
  if (!gate || !up || !out || ldg < cols || ldu < cols || ldo < cols) return QL_EINVAL;
  if (cols % 8 || !rows_ok(gate, ldg, dtype) || !rows_ok(up, ldu, dtype) || !rows_ok(out, ldo, dtype))
    return QL_EALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  QL_DISPATCH_DTYPE(dtype, DT, {
    using T = typename Elem<DT>::T;
    hipLaunchKernelGGL((swiglu_fwd_rows<DT>), dim3(stream_grid(rows * (cols / 8))),
                       dim3(kThreads), 0, s, (const T*)gate, ldg, (const T*)up, ldu, (T*)out, ldo,
                       cols / 8, rows * (cols / 8));
    return ql_launch_status();
  });
  return QL_EDTYPE;
}

extern "C" int qlora_swiglu_bwd_rows(const void* grad, int64_t ldgr, const void* gate, int64_t ldg,
                                     const void* up, int64_t ldu, void* dgate, int64_t lddg,
                                     void* dup, int64_t lddu, int64_t rows, int64_t cols,
                                     int dtype, ql_stream_t stream) {
  if (rows < 0 || cols < 0) return QL_EINVAL;
  if (!ql_valid_dtype(dtype)) return QL_EDTYPE;
  if (rows == 0 || cols == 0) return QL_OK;
  if (!grad || !gate || !up || !dgate || !dup) return QL_EINVAL;
  if (ldgr < cols || ldg < cols || ldu < cols || lddg < cols || lddu < cols) return QL_EINVAL;
  if (cols % 8 || !rows_ok(grad, ldgr, dtype) || !rows_ok(gate, ldg, dtype) ||
      !rows_ok(up, ldu, dtype) || !rows_ok(dgate, lddg, dtype) || !rows_ok(dup, lddu, dtype))
    return QL_EALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  QL_DISPATCH_DTYPE(dtype, DT, {
    using T = typename Elem<DT>::T;
    hipLaunchKernelGGL((swiglu_bwd_rows<DT>), dim3(stream_grid(rows * (cols / 8))),
                       dim3(kThreads), 0, s, (const T*)grad, ldgr, (const T*)gate, ldg,
                       (const T*)up, ldu, (T*)dgate, lddg, (T*)dup, lddu, cols / 8,
                       rows * (cols / 8));
    return ql_launch_status();
  });
  return QL_EDTYPE;
}
