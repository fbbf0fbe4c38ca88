/*
 * quant_ref.c -- plain-C restatement of the two bit-exact quantisers of the
 * lemoq decode path.  TEST INFRASTRUCTURE ONLY (an independent cross-check of
 * oracle/quant.py and of the HIP kernels); never linked into the product.
 *
 *  - oracle_rtn_w8: per-group symmetric RTN, 8-bit
 *      (src/lemoq/quant/numpy_oracle.py:58-116, src/lemoq/quant/rtn.py:68-73):
 *      scale = absmax / 127 in float (1.0f if absmax == 0),
 *      code  = clamp(round_half_even(w / scale), -128, 127).
 *  - oracle_kv_quant_rows: per-token symmetric int8
 *      (src/lemoq/kernels/kv_int8.py:30-41): s = amax / 127 (1.0f if 0),
 *      code = clamp(round_half_even(x / s), -127, 127), scale -> fp16.
 *
 * Built with -O2 -fno-fast-math -ffp-contract=off so every float operation is
 * one IEEE single-precision operation (x86-64 SSE, round to nearest even).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* IEEE binary16 round-to-nearest-even from binary32, written from the format
 * definition (sign, 5-bit exponent with bias 15, 10-bit fraction). */
uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) { /* inf or nan */
    return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
  }
  const int32_t exp = (int32_t)(absx >> 23) - 127;
  uint32_t mant = absx & 0x7fffffu;
  if (exp > 15) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
  if (exp >= -14) {                                 /* normal half */
    uint32_t h = ((uint32_t)(exp + 15) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* may carry into exp: ok */
    return (uint16_t)(sign | h);
  }
  /* subnormal half: value = m * 2^-24 */
  if (exp < -25) return (uint16_t)sign;
  mant |= 0x800000u; /* implicit bit: value = mant * 2^(exp-23) */
  const int drop = -exp - 1; /* value / 2^-24 = mant * 2^(exp+1) */
  uint32_t h = mant >> drop;
  const uint32_t rem = mant & ((1u << drop) - 1u);
  const uint32_t half = 1u << (drop - 1);
  if (rem > half || (rem == half && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

static float round_half_even(float v) { return nearbyintf(v); } /* default FE_TONEAREST */

void oracle_rtn_w8(const float* w, int64_t rows, int64_t cols, int64_t group, int8_t* codes,
                   float* scale32, uint16_t* scale16) {
  const int64_t ng = (cols + group - 1) / group;
  const int64_t padded = ng * group;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < ng; ++g) {
      float amax = 0.0f;
      for (int64_t i = 0; i < group; ++i) {
        const int64_t k = g * group + i;
        const float v = k < cols ? w[r * cols + k] : 0.0f;
        const float a = fabsf(v);
        if (a > amax) amax = a;
      }
      const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
      for (int64_t i = 0; i < group; ++i) {
        const int64_t k = g * group + i;
        const float v = k < cols ? w[r * cols + k] : 0.0f;
        float q = round_half_even(v / s);
        if (q < -128.0f) q = -128.0f;
        if (q > 127.0f) q = 127.0f;
        codes[r * padded + k] = (int8_t)q;
      }
      scale32[r * ng + g] = s;
      scale16[r * ng + g] = oracle_f32_to_f16(s);
    }
  }
}

/* x: rows x d fp16 bit patterns already widened to float by the caller. */
void oracle_kv_quant_rows(const float* x, int64_t rows, int64_t d, int8_t* codes,
                          uint16_t* scale16) {
  for (int64_t r = 0; r < rows; ++r) {
    float amax = 0.0f;
    for (int64_t i = 0; i < d; ++i) {
      const float a = fabsf(x[r * d + i]);
      if (a > amax) amax = a;
    }
    const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    for (int64_t i = 0; i < d; ++i) {
      float q = round_half_even(x[r * d + i] / s);
      if (q < -127.0f) q = -127.0f;
      if (q > 127.0f) q = 127.0f;
      codes[r * d + i] = (int8_t)q;
    }
    scale16[r] = oracle_f32_to_f16(s);
  }
}
