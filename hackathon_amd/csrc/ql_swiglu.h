// SwiGLU math shared by the streaming kernels (swiglu.hip) and the kernel that fuses the
// backward with the adapters' down-projections (lora_mfma.hip), so both compile the same
// expressions and produce the same bits. Reference semantics: solution/swiglu.py:15-37,
// all math in fp32.
#pragma once

#include "ql_common.h"

QL_DEV float ql_sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

// out = gate * sigmoid(gate) * up
QL_DEV float ql_swiglu_fwd1(float g, float u) { return g * ql_sigmoid(g) * u; }

// dup = grad * gate * sig;  dgate = grad * up * sig * (1 + gate * (1 - sig))
QL_DEV void ql_swiglu_bwd1(float gr, float g, float u, float& dg, float& du) {
  const float sg = ql_sigmoid(g);
  du = gr * g * sg;
  dg = gr * u * sg * (1.0f + g * (1.0f - sg));
}
