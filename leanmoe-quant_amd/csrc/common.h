// Shared device helpers for the lemoq gfx950 kernels (wave64, CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lemoq_hip.h"

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define LEMOQ_WAVE 64

// ---------------------------------------------------------------------------
// fp16 <-> fp32.  The f32->f16 conversion is v_cvt_f16_f32 (round to nearest
// even), the same rounding as torch's `.half()` / `.to(torch.float16)`.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(f16, b); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (f16)f); }
// fp16 + fp16 with one rounding, as torch adds two fp16 tensors.
__device__ __forceinline__ uint16_t hadd_round(float a_f16_exact, uint16_t b) {
  return f2h(a_f16_exact + h2f(b));
}

// Reinterpret a dword as an fp16 pair.  Takes the dword BY VALUE on purpose:
// clang's __builtin_bit_cast applied directly to an ext_vector element
// (e.g. `__builtin_bit_cast(f16x2, v.y)` for a u32x4 v) reads element .x
// instead (observed with the ROCm 7.2 clang for gfx950), so vector elements
// must first be copied to a scalar, which this parameter does.
__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }

// ---------------------------------------------------------------------------
// Wave-level reductions (fixed butterfly order => deterministic).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, LEMOQ_WAVE);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, LEMOQ_WAVE));
  return v;
}
// Sum over aligned groups of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, LEMOQ_WAVE);
  return v;
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, LEMOQ_WAVE));
  return v;
}

// ---------------------------------------------------------------------------
// int8 x fp16 dot product of 16 codes.
//
// Four int8 codes c0..c3 packed in a dword become two exact fp16 pairs with
// three bit operations and one packed fp16 subtract:
//   t = c ^ 0x80808080            -> offset-binary bytes u = c + 128
//   (t & 0x00FF00FF) | 0x64006400 -> fp16 pair (1024+u0, 1024+u2)
//   ((t>>8) & 0x00FF00FF) | ...   -> fp16 pair (1024+u1, 1024+u3)
//   pair - 1152                   -> (c0, c2), (c1, c3)   (exact in fp16)
// v_dot2_f32_f16 then forms c*x products exactly in fp32 and accumulates in
// fp32, so the result is the fp32 sum of exact products, as in the
// reference's dequantize-then-multiply loop.  The activation must be given
// pre-permuted: xa = (x0, x2), xb = (x1, x3) for each group of four.
// ---------------------------------------------------------------------------
struct XChunk {  // 16 activations in dot order
  f16x2 a[4];
  f16x2 b[4];
};

__device__ __forceinline__ void load_xchunk(const uint16_t* __restrict__ src, XChunk& xc) {
  // src: 16 consecutive fp16 values (32 bytes, 16-byte aligned), LDS or global.
  const u32x4 p0 = *reinterpret_cast<const u32x4*>(src);
  const u32x4 p1 = *reinterpret_cast<const u32x4*>(src + 8);
  const uint32_t w[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // dword pair (w[2i], w[2i+1]) holds x[4i..4i+3] as (x0|x1<<16, x2|x3<<16)
    const uint32_t lo = w[2 * i], hi = w[2 * i + 1];
    const uint32_t a = (lo & 0xFFFFu) | (hi << 16);          // (x0, x2)
    const uint32_t b = (lo >> 16) | (hi & 0xFFFF0000u);       // (x1, x3)
    xc.a[i] = as_h2(a);
    xc.b[i] = as_h2(b);
  }
}

__device__ __forceinline__ float dot16_i8(const u32x4 c, const XChunk& xc, float acc) {
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  const f16x2 bias = {(f16)1152.0f, (f16)1152.0f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t t = cw[i] ^ 0x80808080u;
    const uint32_t lo = (t & 0x00FF00FFu) | 0x64006400u;
    const uint32_t hi = ((t >> 8) & 0x00FF00FFu) | 0x64006400u;
    const f16x2 clo = as_h2(lo) - bias;
    const f16x2 chi = as_h2(hi) - bias;
    acc = __builtin_amdgcn_fdot2(clo, xc.a[i], acc, false);
    acc = __builtin_amdgcn_fdot2(chi, xc.b[i], acc, false);
  }
  return acc;
}

// 16-byte global load of weights that are streamed once per step.
__device__ __forceinline__ u32x4 load_stream16(const int8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Host-side helpers.
// ---------------------------------------------------------------------------
#define LEMOQ_CHECK_LAUNCH()                          \
  do {                                                \
    hipError_t e__ = hipGetLastError();               \
    return e__ == hipSuccess ? LEMOQ_OK : (int)e__;   \
  } while (0)

static inline bool lemoq_aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}
static inline hipStream_t lemoq_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
