// 8-element vector loads/stores by storage dtype (16 B for 16-bit types, 2 x 16 B for fp32),
// plus uniform-branch scalar access by a runtime dtype tag for the fallback kernels.
#pragma once

#include "ql_common.h"

template <int DT> struct Vec8;

// unpack / pack convert between 8 floats and the 16-byte register image of 8 16-bit values
// (element 2i in the low half of word i).
template <> struct Vec8<QL_BF16> {
  static QL_DEV void unpack(const uint4& r, float* v) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static QL_DEV uint4 pack(const float* v) {
    uint4 r;
    r.x = pack_bf16x2(v[0], v[1]);
    r.y = pack_bf16x2(v[2], v[3]);
    r.z = pack_bf16x2(v[4], v[5]);
    r.w = pack_bf16x2(v[6], v[7]);
    return r;
  }
  static QL_DEV void load(const uint16_t* p, float* v) {
    unpack(*reinterpret_cast<const uint4*>(p), v);
  }
  static QL_DEV void store(uint16_t* p, const float* v) {
    *reinterpret_cast<uint4*>(p) = pack(v);
  }
};

template <> struct Vec8<QL_F16> {
  static QL_DEV void unpack(const uint4& r, float* v) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = f16_bits_to_f32((uint16_t)(w[i] & 0xffffu));
      v[2 * i + 1] = f16_bits_to_f32((uint16_t)(w[i] >> 16));
    }
  }
  static QL_DEV uint4 pack(const float* v) {
    uint4 r;
    r.x = pack_f16x2(v[0], v[1]);
    r.y = pack_f16x2(v[2], v[3]);
    r.z = pack_f16x2(v[4], v[5]);
    r.w = pack_f16x2(v[6], v[7]);
    return r;
  }
  static QL_DEV void load(const uint16_t* p, float* v) {
    unpack(*reinterpret_cast<const uint4*>(p), v);
  }
  static QL_DEV void store(uint16_t* p, const float* v) {
    *reinterpret_cast<uint4*>(p) = pack(v);
  }
};

template <> struct Vec8<QL_F32> {
  static QL_DEV void load(const float* p, float* v) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static QL_DEV void store(float* p, const float* v) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
};

// The register image of 8 elements as loaded (16 B for 16-bit types, 32 B for fp32), kept
// packed until it is unpacked: a kernel can issue every load of a row before its first use
// and hold the row in half the registers 8 floats a chunk would take.
template <int DT> struct Raw8 {
  uint4 r;
  QL_DEV void load(const uint16_t* p) { r = *reinterpret_cast<const uint4*>(p); }
  QL_DEV void load_bytes(const char* p) { r = *reinterpret_cast<const uint4*>(p); }
  QL_DEV void store_bytes(char* p) const { *reinterpret_cast<uint4*>(p) = r; }
  QL_DEV void unpack(float* v) const { Vec8<DT>::unpack(r, v); }
  // An empty register barrier: the value is unchanged, but the compiler must unpack it again
  // afterwards instead of keeping an earlier unpacked copy (8 registers a chunk) alive.
  QL_DEV void opaque() { asm volatile("" : "+v"(r.x), "+v"(r.y), "+v"(r.z), "+v"(r.w)); }
};
template <> struct Raw8<QL_F32> {
  float4 a, b;
  QL_DEV void load(const float* p) {
    a = reinterpret_cast<const float4*>(p)[0];
    b = reinterpret_cast<const float4*>(p)[1];
  }
  QL_DEV void load_bytes(const char* p) { load(reinterpret_cast<const float*>(p)); }
  QL_DEV void store_bytes(char* p) const {
    reinterpret_cast<float4*>(p)[0] = a;
    reinterpret_cast<float4*>(p)[1] = b;
  }
  QL_DEV void unpack(float* v) const {
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  QL_DEV void opaque() {}  // already 8 registers of fp32: nothing to save
};

// Scalar access with a runtime dtype tag (uniform across the wave: no divergence).
QL_DEV float load_any(const void* p, int dt, int64_t i) {
  if (dt == QL_F32) return static_cast<const float*>(p)[i];
  if (dt == QL_F16) return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

QL_DEV void store_any(void* p, int dt, int64_t i, float v) {
  if (dt == QL_F32) static_cast<float*>(p)[i] = v;
  else if (dt == QL_F16) static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
  else static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
}

QL_DEV float round_any(float v, int dt) {
  if (dt == QL_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
  if (dt == QL_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  return v;
}

// torch.promote_types over {f32, f16, bf16}: equal -> itself; any f32 -> f32;
// f16 with bf16 -> f32.
static inline int ql_promote(int a, int b) { return a == b ? a : QL_F32; }

static inline int ql_elem_size(int dt) { return dt == QL_F32 ? 4 : 2; }

static inline bool ql_valid_dtype(int dt) { return dt == QL_F32 || dt == QL_F16 || dt == QL_BF16; }

// Dispatch a (DT_A, DT_B) pair of compile-time dtypes.
#define QL_DISPATCH_DTYPE2(a, b, DA, DB, ...)                    \
  QL_DISPATCH_DTYPE(a, DA, QL_DISPATCH_DTYPE(b, DB, __VA_ARGS__))
