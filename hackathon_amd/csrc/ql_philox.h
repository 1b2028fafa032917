// The LoRA dropout uniform: Philox4x32-10 (Salmon et al., "Parallel Random Numbers: As Easy as
// 1, 2, 3", SC'11) on counter {flat index, 0, 0, 0} and key {seed_lo, seed_hi}, word 0 folded
// to a non-negative int32 (x < 0 -> -x-1) and scaled by 4.6566127342e-10f: the uniform
// Triton's tl.rand(seed, int32 offset) draws (solution/lora.py:41-43), so a seed gives the
// reference's mask. An element is kept when that uniform is > p. Shared by the dropout kernels
// (lora.hip) and the dropout fused with the adapters' down-projections (lora_mfma.hip).
#pragma once

#include "ql_common.h"

namespace ql_philox {

constexpr float kUniformScale = 4.6566127342e-10f;

// Each round's two 32 x 32 -> 64-bit products are written as 64-bit multiplies, so that each
// becomes one v_mad_u64_u32 instead of a v_mul_hi_u32 and a v_mul_lo_u32 (15% faster at
// 4096 x 3584, the same bits), and each three-way xor is one v_bitop3_b32 (truth table 0x96)
// where the compiler would emit two v_xor_b32. The integer work is the dropout kernels' bound.
QL_DEV uint32_t philox_word0(uint32_t ctr, uint64_t seed) {
  uint32_t c0 = ctr, c1 = 0u, c2 = 0u, c3 = 0u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    c0 = __builtin_amdgcn_bitop3_b32(hi1, c1, k0, 0x96);
    c1 = lo1;
    c2 = __builtin_amdgcn_bitop3_b32(hi0, c3, k1, 0x96);
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c0;
}

// The folded word x of the uniform: U = (float)x * kUniformScale.
QL_DEV uint32_t fold_word(uint32_t w) {
  const int32_t x = (int32_t)w;
  return (uint32_t)(x ^ (x >> 31));  // -x - 1 for x < 0 (also for INT32_MIN), else x
}

// keep = U > p. Rounding (float)x and the product are both monotone in x, so U > p holds exactly
// for the folded words x >= keep_threshold(p): the kernels compare integers and skip the
// conversion and the multiply. The threshold is found on the host with the same single-
// precision operations (2^31: nothing is kept).
inline uint32_t keep_threshold(float p) {
  uint64_t lo = 0, hi = uint64_t(1) << 31;
  while (lo < hi) {
    const uint64_t mid = (lo + hi) / 2;
    const float u = (float)(int32_t)mid * kUniformScale;
    if (u > p) hi = mid; else lo = mid + 1;
  }
  return (uint32_t)lo;
}

QL_DEV bool keep_word(uint32_t w, uint32_t threshold) { return fold_word(w) >= threshold; }

// The keep bits of an [M, K] input, in 8 x 8 blocks: the 8 rows 8 R .. 8 R + 7 take
// `group_stride` (>= K) bytes from R * group_stride; in them, the 8 bytes of columns
// 8 b .. 8 b + 7 sit at 8 b, one byte per row (row 8 R + i at 8 b + i), bit j for column
// 8 b + j. An 8 x 8 block is one 8-byte word (the lora_A gradient's transposed reads take it in
// one load), and a 16-row x 64-column tile is 128 contiguous bytes.
QL_DEV int64_t keep_byte(int64_t row, int64_t col, int64_t group_stride) {
  return (row >> 3) * group_stride + (col >> 3) * 8 + (row & 7);
}

}  // namespace ql_philox
