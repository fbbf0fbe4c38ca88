// Matrix-core main loop shared by the multi-token (prefill) GEMMs: a wave
// accumulates a (32*FM) x (32*FN) tile of Y = X W^T with
// v_mfma_f32_32x32x16_f16, X rows fp16 and W rows either w8 (int8 codes +
// fp16 per-group scales, dequantised in registers to fp16(code * scale)) or
// fp16.
//
// Operand layout of v_mfma_f32_32x32x16_f16 (verified on the device): lane l
// holds row (A) / column (B) l % 32 and 8 k-values of the lane half l / 32;
// accumulator register r of lane l is element (8*(r/4) + 4*(l/32) + r%4,
// l % 32).  The sum over k does not depend on which k-values a lane half
// holds as long as A and B agree, so each lane reads 16 consecutive k (one
// 16-byte load of codes, two of fp16) and feeds two instructions: half h takes
// k0 + 16h + [0, 8) in the first and k0 + 16h + [8, 16) in the second.  A
// 32-wide k block lies inside one scale group (group % 32 == 0).
#pragma once

#include "common.h"

namespace lemoq_gemm {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ h8v h8_of(const u32x4 v) { return __builtin_bit_cast(h8v, v); }

// 16 int8 codes (k order) -> two h8v of fp16(code * s): the code becomes an
// exact fp16 through (1024 + (code + 128)) - 1152, and one fp16 multiply
// rounds the exact product once (the fp32 product code * scale is exact, so
// this equals rounding it to fp16).
__device__ __forceinline__ void dequant16(const u32x4 c, uint32_t s2, h8v& lo, h8v& hi) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  const f16x2 sc = as_h2(s2);
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t t = w[i] ^ 0x80808080u;
    const uint32_t p01 = __builtin_amdgcn_perm(0x64646464u, t, 0x04010400u);
    const uint32_t p23 = __builtin_amdgcn_perm(0x64646464u, t, 0x04030402u);
    o[2 * i] = __builtin_bit_cast(uint32_t, (as_h2(p01) - bias) * sc);
    o[2 * i + 1] = __builtin_bit_cast(uint32_t, (as_h2(p23) - bias) * sc);
  }
  lo = __builtin_bit_cast(h8v, (u32x4){o[0], o[1], o[2], o[3]});
  hi = __builtin_bit_cast(h8v, (u32x4){o[4], o[5], o[6], o[7]});
}

// Weight-row source of one B fragment: w8 (codes row + scales row) or fp16.
struct WRow {
  const int8_t* codes;     // row start + 16*half (w8)
  const uint16_t* scale;   // row's scales (w8)
  const uint16_t* w16;     // row start + 16*half (fp16)
};

template <int FM, int FN>
struct Acc {
  f32x16 v[FM][FN];
};

template <int FM, int FN>
__device__ __forceinline__ void acc_zero(Acc<FM, FN>& a) {
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) a.v[i][j] = (f32x16){};
}

// xr[f]: start of the lane's X row for fragment f, already offset by 16*half.
template <bool W8, int FM, int FN>
__device__ __forceinline__ void mainloop(Acc<FM, FN>& acc, const uint16_t* const (&xr)[FM],
                                         const WRow (&wr)[FN], int64_t K, int group) {
  for (int64_t k0 = 0; k0 < K; k0 += 32) {
    u32x4 xa[FM][2];
#pragma unroll
    for (int f = 0; f < FM; ++f) {
      xa[f][0] = *reinterpret_cast<const u32x4*>(xr[f] + k0);
      xa[f][1] = *reinterpret_cast<const u32x4*>(xr[f] + k0 + 8);
    }
    h8v blo[FN], bhi[FN];
    if constexpr (W8) {
      u32x4 wc[FN];
      uint16_t ws[FN];
#pragma unroll
      for (int f = 0; f < FN; ++f) {
        wc[f] = *reinterpret_cast<const u32x4*>(wr[f].codes + k0);
        ws[f] = wr[f].scale[k0 / group];
      }
#pragma unroll
      for (int f = 0; f < FN; ++f) dequant16(wc[f], (uint32_t)ws[f] * 0x10001u, blo[f], bhi[f]);
    } else {
#pragma unroll
      for (int f = 0; f < FN; ++f) {
        blo[f] = h8_of(*reinterpret_cast<const u32x4*>(wr[f].w16 + k0));
        bhi[f] = h8_of(*reinterpret_cast<const u32x4*>(wr[f].w16 + k0 + 8));
      }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h8_of(xa[i][0]), blo[j], acc.v[i][j], 0, 0, 0);
        acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h8_of(xa[i][1]), bhi[j], acc.v[i][j], 0, 0, 0);
      }
  }
}

// Row (within the 32-row fragment) of accumulator register r in lane half `half`.
__device__ __forceinline__ int acc_row(int r, int half) { return 8 * (r / 4) + 4 * half + (r % 4); }

}  // namespace lemoq_gemm
