// Rotary position embedding of q and k in one launch, forward and backward, for gfx950.
//
// Reference semantics: solution/rope.py:24-62 (rope_qk_kernel). With halves (x1, x2) of a
// head vector and (c1, c2), (s1, s2) of cos/sin at the same (batch, position):
//   forward : o1 = x1*c1 - x2*s1          o2 = x2*c2 + x1*s2
//   backward: d1 = g1*c1 + g2*s2          d2 = g2*c2 - g1*s1
// (the backward is the forward with s1 <- -s2, s2 <- -s1; it stays exact when the halves of
// cos/sin differ).
//
// HBM-bound: every element of q and k is read once and written once; cos/sin are read once
// per (batch, position) and reused from registers for every head. One workgroup per
// (batch, position); a work item is (head, 8-dim chunk of the first half), so a thread loads
// 16 B of x1 and 16 B of x2 and stores the same. q and k are (B, H, S, D) with real strides
// (views of (B, S, H, D) buffers), written with the output's own strides.
#include "ql_vec.h"

namespace {

constexpr int kThreads = 256;

struct Strides3 {
  int64_t b, h, s;
};

template <int IT, int CT, int OT, int VW>
__global__ __launch_bounds__(kThreads) void rope_qk_kernel(
    const typename Elem<IT>::T* __restrict__ q, const typename Elem<IT>::T* __restrict__ k,
    typename Elem<OT>::T* __restrict__ qo, typename Elem<OT>::T* __restrict__ ko,
    const typename Elem<CT>::T* __restrict__ cosp, const typename Elem<CT>::T* __restrict__ sinp,
    int64_t S, int HQ, int HK, int half, Strides3 sq, Strides3 sk, Strides3 sqo, Strides3 sko,
    int64_t cs_b, int64_t cs_s, bool backward) {
  const int64_t pid = blockIdx.x;
  const int64_t b = pid / S;
  const int64_t s = pid - b * S;
  const int chunks = half / VW;
  const int items = (HQ + HK) * chunks;
  const auto* cb = cosp + b * cs_b + s * cs_s;
  const auto* sb = sinp + b * cs_b + s * cs_s;
  for (int it = threadIdx.x; it < items; it += kThreads) {
    const int head = it / chunks;
    const int d0 = (it - head * chunks) * VW;
    float c1[VW], c2[VW], s1[VW], s2[VW], x1[VW], x2[VW], o1[VW], o2[VW];
    if constexpr (VW == 8) {
      Vec8<CT>::load(cb + d0, c1);
      Vec8<CT>::load(cb + half + d0, c2);
      Vec8<CT>::load(sb + d0, s1);
      Vec8<CT>::load(sb + half + d0, s2);
    } else {
      c1[0] = Elem<CT>::to_f32(cb[d0]);
      c2[0] = Elem<CT>::to_f32(cb[half + d0]);
      s1[0] = Elem<CT>::to_f32(sb[d0]);
      s2[0] = Elem<CT>::to_f32(sb[half + d0]);
    }
    if (backward) {
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const float t = s1[j];
        s1[j] = -s2[j];
        s2[j] = -t;
      }
    }
    const bool is_q = head < HQ;
    const int h = is_q ? head : head - HQ;
    const Strides3 si = is_q ? sq : sk;
    const Strides3 so = is_q ? sqo : sko;
    const auto* src = (is_q ? q : k) + b * si.b + h * si.h + s * si.s;
    auto* dst = (is_q ? qo : ko) + b * so.b + h * so.h + s * so.s;
    if constexpr (VW == 8) {
      Vec8<IT>::load(src + d0, x1);
      Vec8<IT>::load(src + half + d0, x2);
    } else {
      x1[0] = Elem<IT>::to_f32(src[d0]);
      x2[0] = Elem<IT>::to_f32(src[half + d0]);
    }
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      o1[j] = x1[j] * c1[j] - x2[j] * s1[j];
      o2[j] = x2[j] * c2[j] + x1[j] * s2[j];
    }
    if constexpr (VW == 8) {
      Vec8<OT>::store(dst + d0, o1);
      Vec8<OT>::store(dst + half + d0, o2);
    } else {
      dst[d0] = Elem<OT>::from_f32(o1[0]);
      dst[half + d0] = Elem<OT>::from_f32(o2[0]);
    }
  }
}

bool strides_vec_ok(const Strides3& st, int dt) {
  const int64_t e = ql_elem_size(dt);
  return ((st.b * e) % 16) == 0 && ((st.h * e) % 16) == 0 && ((st.s * e) % 16) == 0;
}

template <int IT, int CT>
int launch_rope(const void* q, const void* k, void* qo, void* ko, const void* c, const void* sn,
                int64_t B, int64_t S, int HQ, int HK, int half, Strides3 sq, Strides3 sk,
                Strides3 sqo, Strides3 sko, int64_t cs_b, int64_t cs_s, bool backward, bool vec,
                hipStream_t st) {
  constexpr int OT = (IT == CT) ? IT : QL_F32;
  using I = typename Elem<IT>::T;
  using C = typename Elem<CT>::T;
  using O = typename Elem<OT>::T;
  const dim3 grid((unsigned)(B * S));
  if (vec)
    hipLaunchKernelGGL((rope_qk_kernel<IT, CT, OT, 8>), grid, dim3(kThreads), 0, st, (const I*)q,
                       (const I*)k, (O*)qo, (O*)ko, (const C*)c, (const C*)sn, S, HQ, HK, half, sq,
                       sk, sqo, sko, cs_b, cs_s, backward);
  else
    hipLaunchKernelGGL((rope_qk_kernel<IT, CT, OT, 1>), grid, dim3(kThreads), 0, st, (const I*)q,
                       (const I*)k, (O*)qo, (O*)ko, (const C*)c, (const C*)sn, S, HQ, HK, half, sq,
                       sk, sqo, sko, cs_b, cs_s, backward);
  return ql_launch_status();
}

}  // namespace

extern "C" int qlora_rope_qk(const void* q, const void* k, void* q_out, void* k_out,
                             const void* cos, const void* sin, int in_dtype, int cs_dtype,
                             int out_dtype, int64_t B, int64_t S, int64_t HQ, int64_t HK,
                             int64_t D, const int64_t* q_strides, const int64_t* k_strides,
                             const int64_t* qo_strides, const int64_t* ko_strides,
                             int64_t cs_stride_b, int64_t cs_stride_s, int backward,
                             ql_stream_t stream) {
  if (B < 0 || S < 0 || HQ < 0 || HK < 0 || D <= 0 || (D & 1)) return QL_EINVAL;
  if (!ql_valid_dtype(in_dtype) || !ql_valid_dtype(cs_dtype) ||
      out_dtype != ql_promote(in_dtype, cs_dtype))
    return QL_EDTYPE;
  if (B * S == 0 || HQ + HK == 0) return QL_OK;
  if (!q_strides || !k_strides || !qo_strides || !ko_strides) return QL_EINVAL;
  if ((HQ && (!q || !q_out)) || (HK && (!k || !k_out)) || !cos || !sin) return QL_EINVAL;
  if (B * S > INT32_MAX || HQ > 65536 || HK > 65536) return QL_EINVAL;
  const Strides3 sq{q_strides[0], q_strides[1], q_strides[2]};
  const Strides3 sk{k_strides[0], k_strides[1], k_strides[2]};
  const Strides3 sqo{qo_strides[0], qo_strides[1], qo_strides[2]};
  const Strides3 sko{ko_strides[0], ko_strides[1], ko_strides[2]};
  const int half = (int)(D / 2);
  const int64_t ce = ql_elem_size(cs_dtype);
  const bool vec = (half % 8) == 0 && strides_vec_ok(sq, in_dtype) && strides_vec_ok(sk, in_dtype) &&
                   strides_vec_ok(sqo, out_dtype) && strides_vec_ok(sko, out_dtype) &&
                   (!HQ || (ql_aligned(q, 16) && ql_aligned(q_out, 16))) &&
                   (!HK || (ql_aligned(k, 16) && ql_aligned(k_out, 16))) && ql_aligned(cos, 16) &&
                   ql_aligned(sin, 16) && ((cs_stride_b * ce) % 16) == 0 &&
                   ((cs_stride_s * ce) % 16) == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  QL_DISPATCH_DTYPE2(in_dtype, cs_dtype, IT, CT,
                     return launch_rope<IT, CT>(q, k, q_out, k_out, cos, sin, B, S, (int)HQ,
                                                (int)HK, half, sq, sk, sqo, sko, cs_stride_b,
                                                cs_stride_s, backward != 0, vec, st));
  return QL_EDTYPE;
}
