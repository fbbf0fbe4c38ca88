// 4-bit code and activation helpers shared by the weight-format GEMV
// (quant_formats.hip) and the 4-bit grouped MoE (moe_q4.hip).
#pragma once

#include "common.h"

namespace lemoq_qf {

// Activation slice of one lane for chunk j: NV values from k0, zero at or past K.
template <int NV>
__device__ __forceinline__ void xq_load(uint32_t (&w)[NV / 2], const uint16_t* __restrict__ xr, int K, int k0,
                                        bool vec) {
  if (vec && k0 + NV <= K) {
#pragma unroll
    for (int q = 0; q < NV / 8; ++q) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(xr + k0 + 8 * q);
      w[4 * q + 0] = v.x;
      w[4 * q + 1] = v.y;
      w[4 * q + 2] = v.z;
      w[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NV / 2; ++i) {
      const int e = k0 + 2 * i;
      const uint32_t lo = e < K ? xr[e] : 0u;
      const uint32_t hi = e + 1 < K ? xr[e + 1] : 0u;
      w[i] = lo | (hi << 16);
    }
  }
}

// 16 values in natural pairs (8 dwords) -> XChunk (dot order of dot16_*):
// one byte permute per pair, a = (x0, x2) and b = (x1, x3) of each four.
__device__ __forceinline__ void xchunk_of(const uint32_t* w, XChunk& xc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = w[2 * i], hi = w[2 * i + 1];
    xc.a[i] = as_h2(__builtin_amdgcn_perm(hi, lo, 0x05040100u));
    xc.b[i] = as_h2(__builtin_amdgcn_perm(hi, lo, 0x07060302u));
  }
}

// 32 packed 4-bit codes (16 bytes; byte b of dword d holds codes 8d + 2b in
// its low nibble and 8d + 2b + 1 in its high nibble) x 32 activations given as
// two XChunks (x[0, 16) and x[16, 32)).  SIGNED: int4 -8 .. 7 (xor 8 gives the
// offset-binary nibble n + 8, minus 1032); else uint4 0 .. 15 (minus 1024).
// Low nibbles of a dword are the codes (8d, 8d+2, 8d+4, 8d+6), high nibbles
// (8d+1, 8d+3, 8d+5, 8d+7): the (x0, x2) / (x1, x3) pairs of XChunk.
// (Placing each nibble position under its own fp16 exponent with one and-or
// per pair instead of the byte permutes measured no faster.)
template <bool SIGNED>
__device__ __forceinline__ float dot32_i4(const u32x4 c, const XChunk& x0, const XChunk& x1, float acc) {
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  const f16x2 bias = SIGNED ? (f16x2){(f16)1032.0f, (f16)1032.0f} : (f16x2){(f16)1024.0f, (f16)1024.0f};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t t = SIGNED ? cw[d] ^ 0x88888888u : cw[d];
    const uint32_t lo = t & 0x0F0F0F0Fu, hi = (t >> 4) & 0x0F0F0F0Fu;
    const XChunk& xc = d < 2 ? x0 : x1;
    const int i0 = 2 * (d & 1);
    const f16x2 p0 = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u)) - bias;  // 8d, 8d+2
    const f16x2 p1 = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u)) - bias;  // 8d+4, 8d+6
    const f16x2 p2 = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u)) - bias;  // 8d+1, 8d+3
    const f16x2 p3 = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u)) - bias;  // 8d+5, 8d+7
    acc = __builtin_amdgcn_fdot2(p0, xc.a[i0], acc, false);
    acc = __builtin_amdgcn_fdot2(p1, xc.a[i0 + 1], acc, false);
    acc = __builtin_amdgcn_fdot2(p2, xc.b[i0], acc, false);
    acc = __builtin_amdgcn_fdot2(p3, xc.b[i0 + 1], acc, false);
  }
  return acc;
}

}  // namespace lemoq_qf
