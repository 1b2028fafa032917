// SwiGLU math shared by the streaming kernels (swiglu.hip) and the kernel that fuses the
// backward with the adapters' down-projections (lora_mfma.hip), so both compile the same
// expressions and produce the same bits. Reference semantics: solution/swiglu.py:15-37,
// all math in fp32.
#pragma once

#include "ql_common.h"

// sigmoid(x) = 1 / (1 + exp(-x)), the division correctly rounded in fp32.
//
// For d = 1 + exp(-x) in [1, 2^126) the correctly rounded 1 / d is the hardware reciprocal
// (v_rcp_f32, within 1 ulp) after one Newton correction in fused multiply-adds,
// r + fma(-d, r, 1) * r. That holds for every one of the 1,056,964,608 fp32 values in the
// range on gfx950 (the exhaustive check of tests/test_gpu_sigmoid_recip.py), and costs 3
// instructions against about 10 for the division sequence hipcc emits, the largest part of
// the SwiGLU backward's arithmetic. Above 2^126 (denormal results; +inf for x < -88.7) and
// for NaN the correction is wrong, and the division is used. The kernels choose on the
// inputs: x > -87 keeps d below 2^126 (exp(87) < 2^125.6) and fails for NaN, so a workgroup
// tests its gate values once and runs one of two copies of its arithmetic.
QL_DEV float ql_recip_fast(float d) {
  const float r = __builtin_amdgcn_rcpf(d);
  return __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
}
QL_DEV bool ql_sigmoid_fast_ok(float x) { return x > -87.0f; }

template <bool FAST> QL_DEV float ql_sigmoid_as(float x) {
  const float d = 1.0f + __expf(-x);
  return FAST ? ql_recip_fast(d) : 1.0f / d;
}
QL_DEV float ql_sigmoid(float x) {
  return ql_sigmoid_fast_ok(x) ? ql_sigmoid_as<true>(x) : ql_sigmoid_as<false>(x);
}
QL_DEV bool ql_sigmoid_fast_ok8(const float* x) {
  bool ok = true;
#pragma unroll
  for (int e = 0; e < 8; ++e) ok &= ql_sigmoid_fast_ok(x[e]);
  return ok;
}

// out = gate * sigmoid(gate) * up
QL_DEV float ql_swiglu_fwd1(float g, float u) { return g * ql_sigmoid(g) * u; }
template <bool FAST> QL_DEV void ql_swiglu_fwd8_as(const float* g, const float* u, float* o) {
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = g[e] * ql_sigmoid_as<FAST>(g[e]) * u[e];
}
QL_DEV void ql_swiglu_fwd8(const float* g, const float* u, float* o) {  // one branch per 8
  if (__builtin_expect(ql_sigmoid_fast_ok8(g), 1)) ql_swiglu_fwd8_as<true>(g, u, o);
  else ql_swiglu_fwd8_as<false>(g, u, o);
}

// dup = grad * gate * sig;  dgate = grad * up * sig * (1 + gate * (1 - sig))
QL_DEV void ql_swiglu_bwd_sig(float gr, float g, float u, float sg, float& dg, float& du) {
  du = gr * g * sg;
  dg = gr * u * sg * (1.0f + g * (1.0f - sg));
}
QL_DEV void ql_swiglu_bwd1(float gr, float g, float u, float& dg, float& du) {
  ql_swiglu_bwd_sig(gr, g, u, ql_sigmoid(g), dg, du);
}
template <bool FAST>
QL_DEV void ql_swiglu_bwd8_as(const float* gr, const float* g, const float* u, float* dg,
                              float* du) {
#pragma unroll
  for (int e = 0; e < 8; ++e)
    ql_swiglu_bwd_sig(gr[e], g[e], u[e], ql_sigmoid_as<FAST>(g[e]), dg[e], du[e]);
}
QL_DEV void ql_swiglu_bwd8(const float* gr, const float* g, const float* u, float* dg,
                           float* du) {  // one branch per 8
  if (__builtin_expect(ql_sigmoid_fast_ok8(g), 1)) ql_swiglu_bwd8_as<true>(gr, g, u, dg, du);
  else ql_swiglu_bwd8_as<false>(gr, g, u, dg, du);
}
