/*
 * CPU oracle (test infrastructure only): NF4 dequantisation, restated in plain C from the
 * reference's kernel, solution/nf4.py:25-49, and its host unpacking, solution/nf4.py:71-92.
 *
 *   weight j lives in packed byte j/2: high nibble for even j, low nibble for odd j (:30,45-47)
 *   block b = j / blocksize (:37)
 *   nested : s = code2[absmax_q[b]] * absmax2[b / blocksize2];  s = s + offset   (:39-42)
 *   plain  : s = absmax[b]                                                        (:44)
 *   out[j] = nf4[nibble] * s  in fp32, then rounded once to the output type      (:45-48)
 *
 * Built with -ffp-contract=off so each * and + rounds separately, and the bf16 rounding is
 * written out here (round to nearest, ties to even), independent of any GPU toolchain.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline use this file.
 */
#include <stdint.h>
#include <string.h>

static float scale_of(int64_t b, int nested, const void* absmax, const float* code2,
                      const float* absmax2, float offset, int64_t blocksize2) {
  if (nested) {
    const uint8_t q = ((const uint8_t*)absmax)[b];
    float s = code2[q] * absmax2[b / blocksize2];
    s = s + offset;
    return s;
  }
  return ((const float*)absmax)[b];
}

uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
  const uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

/* fp32 results (before the final rounding) */
void oracle_nf4_dequant_f32(const uint8_t* packed, int64_t n_weights, const void* absmax,
                            int nested, const float* code2, const float* absmax2, float offset,
                            int64_t blocksize, int64_t blocksize2, const float* table,
                            float* out) {
  for (int64_t j = 0; j < n_weights; ++j) {
    const uint8_t byte = packed[j >> 1];
    const unsigned nib = (j & 1) ? (byte & 15u) : (byte >> 4);
    const float s = scale_of(j / blocksize, nested, absmax, code2, absmax2, offset, blocksize2);
    out[j] = table[nib] * s;
  }
}

/* bf16 results: the fp32 product rounded once, RNE */
void oracle_nf4_dequant_bf16(const uint8_t* packed, int64_t n_weights, const void* absmax,
                             int nested, const float* code2, const float* absmax2, float offset,
                             int64_t blocksize, int64_t blocksize2, const float* table,
                             uint16_t* out) {
  for (int64_t j = 0; j < n_weights; ++j) {
    const uint8_t byte = packed[j >> 1];
    const unsigned nib = (j & 1) ? (byte & 15u) : (byte >> 4);
    const float s = scale_of(j / blocksize, nested, absmax, code2, absmax2, offset, blocksize2);
    out[j] = oracle_f32_to_bf16(table[nib] * s);
  }
}

/* the block scales alone (the double-quant reconstruction) */
void oracle_nf4_scales(int64_t n_blocks, const void* absmax, int nested, const float* code2,
                       const float* absmax2, float offset, int64_t blocksize2, float* out) {
  for (int64_t b = 0; b < n_blocks; ++b)
    out[b] = scale_of(b, nested, absmax, code2, absmax2, offset, blocksize2);
}
