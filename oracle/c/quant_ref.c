/*
 * quant_ref.c -- plain-C restatement of the bit-exact quantisers of the
 * lemoq decode path and of its weight formats.  TEST INFRASTRUCTURE ONLY (an independent cross-check of
 * oracle/quant.py and of the HIP kernels); never linked into the product.
 *
 *  - oracle_rtn_w8: per-group symmetric RTN, 8-bit
 *      (src/lemoq/quant/numpy_oracle.py:58-116, src/lemoq/quant/rtn.py:68-73):
 *      scale = absmax / 127 in float (1.0f if absmax == 0),
 *      code  = clamp(round_half_even(w / scale), -128, 127).
 *  - oracle_kv_quant_rows: per-token symmetric int8
 *      (src/lemoq/kernels/kv_int8.py:30-41): s = amax / 127 (1.0f if 0),
 *      code = clamp(round_half_even(x / s), -127, 127), scale -> fp16.
 *  - oracle_rtn: per-group RTN at 4 or 8 bits, symmetric or asymmetric.
 *  - oracle_mxfp4: the MXFP4 (E2M1 + E8M0) quantiser.
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

/* Per-group RTN at 4 or 8 bits, symmetric or asymmetric
 * (src/lemoq/quant/numpy_oracle.py:58-107): codes as int32 (rows, padded),
 * scale and zero as float (rows, ng).  Asymmetric min/max skip the zero
 * padding of the last group. */
void oracle_rtn(const float* w, int64_t rows, int64_t cols, int64_t group, int bits, int symmetric,
                int32_t* codes, float* scale32, float* zero32) {
  const int64_t ng = (cols + group - 1) / group;
  const int64_t padded = ng * group;
  const float qmax = symmetric ? (float)((1 << (bits - 1)) - 1) : (float)((1 << bits) - 1);
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < ng; ++g) {
      float s, z = 0.0f;
      if (symmetric) {
        float amax = 0.0f;
        for (int64_t i = 0; i < group; ++i) {
          const int64_t k = g * group + i;
          const float a = fabsf(k < cols ? w[r * cols + k] : 0.0f);
          if (a > amax) amax = a;
        }
        s = amax > 0.0f ? amax / qmax : 1.0f;
      } else {
        float gmax = -INFINITY, gmin = INFINITY;
        for (int64_t i = 0; i < group; ++i) {
          const int64_t k = g * group + i;
          if (k >= cols) break;
          const float v = w[r * cols + k];
          if (v > gmax) gmax = v;
          if (v < gmin) gmin = v;
        }
        if (!isfinite(gmax)) gmax = 0.0f;
        if (!isfinite(gmin)) gmin = 0.0f;
        const float rng = gmax - gmin;
        s = rng > 0.0f ? rng / qmax : 1.0f;
        z = round_half_even(-gmin / s);
      }
      const float lo = symmetric ? -(qmax + 1.0f) : 0.0f;
      for (int64_t i = 0; i < group; ++i) {
        const int64_t k = g * group + i;
        float q = round_half_even((k < cols ? w[r * cols + k] : 0.0f) / s);
        if (!symmetric) q = q + z;
        if (q < lo) q = lo;
        if (q > qmax) q = qmax;
        codes[r * padded + k] = (int32_t)q;
      }
      scale32[r * ng + g] = s;
      zero32[r * ng + g] = z;
    }
  }
}

/* MXFP4 (src/lemoq/quant/mxfp4.py:50-102): per block of 32 (zero padded),
 * X = floor of log2(amax) rounded to float (computed in long double here),
 * minus 2, clamped to [-127, 127] (-127 for an all-zero block); v = w / 2^X;
 * magnitude code = first nearest of {0,.5,1,1.5,2,3,4,6} to min(|v|, 6);
 * sign bit v < 0.  codes (rows, nblk*32) unpacked, scale bytes (rows, nblk). */
void oracle_mxfp4(const float* w, int64_t rows, int64_t cols, uint8_t* codes, uint8_t* scales) {
  static const float mags[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const int64_t nblk = (cols + 31) / 32;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t b = 0; b < nblk; ++b) {
      float amax = 0.0f;
      for (int i = 0; i < 32; ++i) {
        const int64_t k = b * 32 + i;
        const float a = fabsf(k < cols ? w[r * cols + k] : 0.0f);
        if (a > amax) amax = a;
      }
      float X = -127.0f;
      if (amax > 0.0f) {
        const float l = (float)log2l((long double)amax);
        X = floorf(l) - 2.0f;
        if (X < -127.0f) X = -127.0f;
        if (X > 127.0f) X = 127.0f;
      }
      const float scale = ldexpf(1.0f, (int)X);
      scales[r * nblk + b] = (uint8_t)(int)(X + 127.0f);
      for (int i = 0; i < 32; ++i) {
        const int64_t k = b * 32 + i;
        const float v = (k < cols ? w[r * cols + k] : 0.0f) / scale;
        float m = fabsf(v);
        if (m > 6.0f) m = 6.0f;
        int best = 0;
        float bd = fabsf(m - mags[0]);
        for (int j = 1; j < 8; ++j) {
          const float d = fabsf(m - mags[j]);
          if (d < bd) {
            bd = d;
            best = j;
          }
        }
        codes[r * nblk * 32 + b * 32 + i] = (uint8_t)((v < 0.0f ? 8 : 0) | best);
      }
    }
  }
}
