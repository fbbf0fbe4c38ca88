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
//
// f2h first pins its argument as an fp32 register value.  Without that, the
// compiler (fp-contract=fast, hipcc's default) folds the fp32 multiply or fma
// that produced the argument and the conversion into one mixed-precision op
// (v_fma_mixlo_f16), which rounds the exact product once to fp16, where the
// reference rounds it to fp32 first and then to fp16 (`(x * rstd).to(fp16)`
// in fp32 arithmetic).  The two differ when the fp32 rounding lands the
// product on an fp16 rounding tie: rare, but enough to move single elements
// of a normalised row by one fp16 ulp, and the fold is applied to some
// elements of a row and not to others depending on the surrounding code.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(f16, b); }
__device__ __forceinline__ uint16_t f2h(float f) {
  __asm__("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (f16)f);
}
// fp16 + fp16 with one rounding, as torch adds two fp16 tensors.
__device__ __forceinline__ uint16_t hadd_round(float a_f16_exact, uint16_t b) {
  return f2h(a_f16_exact + h2f(b));
}

// HF OLMoE's clip_qkv on one fp16 value (torch's clamp_(min=-c, max=c) of
// the normed q, the normed k and the raw v rows): a value above c becomes
// c16 = fp16(c), below -c becomes -c16, NaN passes through (both comparisons
// are false).  c = +inf leaves every value as it is.
__device__ __forceinline__ float clip_qkv(float x, float c, float c16) {
  return x > c ? c16 : (x < -c ? -c16 : x);
}

// Reinterpret a dword as an fp16 pair.  Takes the dword BY VALUE on purpose:
// clang's __builtin_bit_cast applied directly to an ext_vector element
// (e.g. `__builtin_bit_cast(f16x2, v.y)` for a u32x4 v) reads element .x
// instead (observed with the ROCm 7.2 clang for gfx950), so vector elements
// must first be copied to a scalar, which this parameter does.
__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ float as_f32(uint32_t v) { return __builtin_bit_cast(float, v); }  // same rule

// ---------------------------------------------------------------------------
// Wave-level reductions, deterministic (fixed combination order).
// Within each row of 16 lanes: DPP quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror leave the row's total in every lane of the row;
// the four row totals are then combined through v_readlane in row order, so
// the result is wave-uniform.  No LDS traffic (a ds_bpermute butterfly costs
// an LDS round trip per step).
// ---------------------------------------------------------------------------
#define LEMOQ_DPP_QUAD_1032 0xB1
#define LEMOQ_DPP_QUAD_2301 0x4E
#define LEMOQ_DPP_ROW_HALF_MIRROR 0x141
#define LEMOQ_DPP_ROW_MIRROR 0x140

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<LEMOQ_DPP_QUAD_1032>(v);
  v += dpp_f<LEMOQ_DPP_QUAD_2301>(v);
  v += dpp_f<LEMOQ_DPP_ROW_HALF_MIRROR>(v);
  v += dpp_f<LEMOQ_DPP_ROW_MIRROR>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
// Block-wide sum over 256 threads (4 waves); every thread gets the total.
__device__ __forceinline__ float block_sum_256(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float t = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return t;
}

// One row of RMSNorm by a 256-thread block, with the rounding points of HF
// OlmoeRMSNorm.forward (src/lemoq/kernels/rmsnorm.py:184-202): fp32 mean of
// squares (thread t sums columns t, t + 256, ... in order, then the block
// sum), x * rstd rounded to fp16, then the fp16 product with the weight.
// xr may point to global memory or LDS; the result does not depend on which.
__device__ __forceinline__ void rmsnorm_row_256(const uint16_t* xr, int H, const uint16_t* __restrict__ w,
                                                float eps, uint16_t* __restrict__ yr, float* red) {
  float ssq = 0.0f;
  for (int i = threadIdx.x; i < H; i += 256) {
    const float a = h2f(xr[i]);
    ssq += a * a;
  }
  const float tot = block_sum_256(ssq, red);
  const float rstd = 1.0f / sqrtf(tot / (float)H + eps);
  for (int i = threadIdx.x; i < H; i += 256) {
    const uint16_t nh = f2h(h2f(xr[i]) * rstd);
    yr[i] = f2h(h2f(nh) * h2f(w[i]));
  }
}

// The same RMSNorm on a row held in registers: thread t of the 256 owns the
// 16-byte chunks at columns 8 (t + 256 i), i < RN_CHUNKS, those below H
// (H % 8 == 0, H <= 2048 * RN_CHUNKS, rows and w 16-byte aligned).  Thread t
// sums its chunks' squares in column order, then the block sum; every caller
// of this function on the same row gets the same bits.
constexpr int RN_CHUNKS = 4;
__device__ __forceinline__ void rmsnorm_chunks(const u32x4 (&x)[RN_CHUNKS], int H, const uint16_t* __restrict__ w,
                                               float eps, uint16_t* __restrict__ yr, float* red) {
  const int c0 = 8 * (int)threadIdx.x;
  u32x4 wv[RN_CHUNKS];
#pragma unroll
  for (int i = 0; i < RN_CHUNKS; ++i)
    if (c0 + 2048 * i < H) wv[i] = *reinterpret_cast<const u32x4*>(w + c0 + 2048 * i);
  float ssq = 0.0f;
#pragma unroll
  for (int i = 0; i < RN_CHUNKS; ++i) {
    if (c0 + 2048 * i >= H) continue;
    const uint32_t q[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a = h2f((uint16_t)(q[k] & 0xFFFFu)), b = h2f((uint16_t)(q[k] >> 16));
      ssq += a * a;
      ssq += b * b;
    }
  }
  const float tot = block_sum_256(ssq, red);
  const float rstd = 1.0f / sqrtf(tot / (float)H + eps);
#pragma unroll
  for (int i = 0; i < RN_CHUNKS; ++i) {
    if (c0 + 2048 * i >= H) continue;
    const uint32_t q[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
    const uint32_t g[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t na = f2h(h2f((uint16_t)(q[k] & 0xFFFFu)) * rstd);
      const uint16_t nb = f2h(h2f((uint16_t)(q[k] >> 16)) * rstd);
      const uint16_t ya = f2h(h2f(na) * h2f((uint16_t)(g[k] & 0xFFFFu)));
      const uint16_t yb = f2h(h2f(nb) * h2f((uint16_t)(g[k] >> 16)));
      o[k] = (uint32_t)ya | ((uint32_t)yb << 16);
    }
    *reinterpret_cast<u32x4*>(yr + c0 + 2048 * i) = (u32x4){o[0], o[1], o[2], o[3]};
  }
}

// The chunks of rmsnorm_chunks from a row in global memory or LDS.
__device__ __forceinline__ void rmsnorm_load_chunks(const uint16_t* xr, int H, u32x4 (&x)[RN_CHUNKS]) {
  const int c0 = 8 * (int)threadIdx.x;
#pragma unroll
  for (int i = 0; i < RN_CHUNKS; ++i)
    if (c0 + 2048 * i < H) x[i] = *reinterpret_cast<const u32x4*>(xr + c0 + 2048 * i);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<LEMOQ_DPP_QUAD_1032>(v));
  v = fmaxf(v, dpp_f<LEMOQ_DPP_QUAD_2301>(v));
  v = fmaxf(v, dpp_f<LEMOQ_DPP_ROW_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_f<LEMOQ_DPP_ROW_MIRROR>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
// Cross-row exchanges of gfx950 (v_permlane16_swap / v_permlane32_swap, no
// LDS): the value of lane ^ 16 or lane ^ 32.  The swap returns both halves;
// the partner is selected by lane.  (Adding the two returned halves directly
// is miscompiled when both operands are the same value: the compiler adds
// one half to itself.  Selecting the partner and adding it to the lane's own
// value is exact and symmetric: both lanes of a pair hold the same sum.)
__device__ __forceinline__ float xor16_get(float v, int lane) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v),
                                                  __builtin_bit_cast(uint32_t, v), false, false);
  return __builtin_bit_cast(float, (lane & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32_get(float v, int lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v),
                                                  __builtin_bit_cast(uint32_t, v), false, false);
  return __builtin_bit_cast(float, lane < 32 ? r[1] : r[0]);
}

#define LEMOQ_DPP_ROW_ROR4 0x124
#define LEMOQ_DPP_ROW_ROR8 0x128

// Sum over the lanes that share lane % G (G in {4, 8, 16}): the total of the
// 64 / G groups of G lanes, in every lane.  Row rotations by 4 and 8 (DPP),
// then the two cross-row swaps; no LDS.
template <int G>
__device__ __forceinline__ float group_total(float v, int lane) {
  static_assert(G == 4 || G == 8 || G == 16, "G must be 4, 8 or 16");
  if (G == 4) v += dpp_f<LEMOQ_DPP_ROW_ROR4>(v);
  if (G <= 8) v += dpp_f<LEMOQ_DPP_ROW_ROR8>(v);
  v += xor16_get(v, lane);
  return v + xor32_get(v, lane);
}

// Sum of squares of 8 fp16 values (16 bytes) added to acc: four v_dot2_f32_f16
// (x.lo^2 + x.hi^2 + acc, products exact in fp32) in word order.
__device__ __forceinline__ float ssq_f16x8(u32x4 v, float acc) {
  acc = __builtin_amdgcn_fdot2(as_h2(v.x), as_h2(v.x), acc, false);
  acc = __builtin_amdgcn_fdot2(as_h2(v.y), as_h2(v.y), acc, false);
  acc = __builtin_amdgcn_fdot2(as_h2(v.z), as_h2(v.z), acc, false);
  return __builtin_amdgcn_fdot2(as_h2(v.w), as_h2(v.w), acc, false);
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
// one xor, two byte permutes and two packed fp16 subtracts:
//   t = c ^ 0x80808080            -> offset-binary bytes u = c + 128
//   perm(0x64.., t) bytes (u0,0x64,u2,0x64) -> fp16 pair (1024+u0, 1024+u2)
//   perm(0x64.., t) bytes (u1,0x64,u3,0x64) -> fp16 pair (1024+u1, 1024+u3)
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
    const uint32_t t = cw[i] ^ 0x80808080u;  // offset-binary bytes u = c + 128
    // v_perm_b32 byte select over {0x64646464 (bytes 4-7), t (bytes 0-3)}:
    // lo = bytes (u0, 0x64, u2, 0x64), hi = bytes (u1, 0x64, u3, 0x64)
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, t, 0x04020400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, t, 0x04030401u);
    const f16x2 clo = as_h2(lo) - bias;
    const f16x2 chi = as_h2(hi) - bias;
    acc = __builtin_amdgcn_fdot2(clo, xc.a[i], acc, false);
    acc = __builtin_amdgcn_fdot2(chi, xc.b[i], acc, false);
  }
  return acc;
}

// Build the dot-order chunk from 16 consecutive fp16 values held in two
// dwordx4 registers (same permutation as load_xchunk).
__device__ __forceinline__ void make_xchunk(const u32x4 p0, const u32x4 p1, XChunk& xc) {
  const uint32_t w[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = w[2 * i], hi = w[2 * i + 1];
    xc.a[i] = as_h2((lo & 0xFFFFu) | (hi << 16));
    xc.b[i] = as_h2((lo >> 16) | (hi & 0xFFFF0000u));
  }
}

// 16-byte global load of weights that are streamed once per step.
__device__ __forceinline__ u32x4 load_stream16(const int8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Loads-first streaming of int8 weight rows.
//
// A row of Kp int8 codes is read as ceil(Kp/1024) chunks of 1 KB; lane l owns
// bytes [1024*j + 16*l, +16) of chunk j, so its 16 codes lie inside one
// quantisation group (group % 16 == 0) and need one fp16 scale.  w8_issue
// only issues the loads (codes and scales of R rows); callers issue every
// other independent load next and only then start arithmetic, so each lane
// keeps R*KCH 16-byte loads in flight from the first cycles of the kernel.
// ---------------------------------------------------------------------------
template <int R, int KCH>
struct W8Tile {
  u32x4 c[R][KCH];
  uint16_t s[R][KCH];
  uint32_t ok;  // bit r*KCH + j: slice (r, j) lies inside the matrix
};

// EXACT: every row of the tile exists and Kp == 1024*KCH, so the loads are
// straight-line code.  Otherwise addresses are clamped into the matrix (no
// branch around a load, which would make the compiler wait on each one) and
// the slices outside it are zeroed through `ok` when they are used.
template <int R, int KCH, bool EXACT>
__device__ __forceinline__ void w8_issue(W8Tile<R, KCH>& t, const int8_t* __restrict__ codes,
                                         const uint16_t* __restrict__ scale, int64_t row0,
                                         int64_t nrows, int Kp, int ngroups, int group,
                                         int lane) {
  t.ok = 0u;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = row0 + r;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int off = 1024 * j + 16 * lane;
      if constexpr (EXACT) {
        t.c[r][j] = load_stream16(codes + row * Kp + off);
        t.s[r][j] = scale[row * ngroups + off / group];
        t.ok |= 1u << (r * KCH + j);
      } else {
        const bool in = row < nrows && off < Kp;
        const int64_t rr = in ? row : 0;
        const int oo = in ? off : 0;
        t.c[r][j] = load_stream16(codes + rr * Kp + oo);
        t.s[r][j] = scale[rr * ngroups + oo / group];
        t.ok |= (in ? 1u : 0u) << (r * KCH + j);
      }
    }
  }
}

// sum_j scale_j * (codes_j . x_j) for row r of the tile.
template <int R, int KCH>
__device__ __forceinline__ float w8_row_dot(const W8Tile<R, KCH>& t, int r, const XChunk (&xc)[KCH]) {
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < KCH; ++j) {
    const float sc = ((t.ok >> (r * KCH + j)) & 1u) ? h2f(t.s[r][j]) : 0.0f;
    a = fmaf(sc, dot16_i8(t.c[r][j], xc[j], 0.0f), a);
  }
  return a;
}

// sum_j x_j . fp16(codes_j * scale_j) for row r of the tile: the weights
// rounded to fp16 first, as a multi-token linear's dequantise-then-GEMM does
// (fp16(code * scale) with one rounding: the code is exact in fp16 and the
// fp16 multiply rounds the product once), then fp32 dot products.
template <int R, int KCH>
__device__ __forceinline__ float w8_row_dot_dq(const W8Tile<R, KCH>& t, int r, const XChunk (&xc)[KCH]) {
  float a = 0.0f;
  const f16x2 bias = {(f16)1152.0f, (f16)1152.0f};
#pragma unroll
  for (int j = 0; j < KCH; ++j) {
    if (!((t.ok >> (r * KCH + j)) & 1u)) continue;
    const f16x2 sc = as_h2((uint32_t)t.s[r][j] * 0x10001u);
    const uint32_t cw[4] = {t.c[r][j].x, t.c[r][j].y, t.c[r][j].z, t.c[r][j].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t u = cw[i] ^ 0x80808080u;
      const f16x2 wlo = (as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04020400u)) - bias) * sc;
      const f16x2 whi = (as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030401u)) - bias) * sc;
      a = __builtin_amdgcn_fdot2(wlo, xc[j].a[i], a, false);
      a = __builtin_amdgcn_fdot2(whi, xc[j].b[i], a, false);
    }
  }
  return a;
}

// The activation slice of one lane: 16 fp16 values per 1 KB chunk, raw bits.
template <int KCH>
struct XRaw {
  u32x4 v[KCH][2];
};

// Issue the loads of src[1024*j + 16*lane, +16) for every chunk.
// EXACT: n == 1024*KCH and src 16-byte aligned (straight-line vector loads).
// Otherwise elements at or beyond n read as 0; `vec` (uniform) says src is
// 16-byte aligned and n % 8 == 0, so whole in-range slices use vector loads.
template <int KCH, bool EXACT>
__device__ __forceinline__ void x_issue(XRaw<KCH>& x, const uint16_t* __restrict__ src, int n,
                                        bool vec, int lane) {
#pragma unroll
  for (int j = 0; j < KCH; ++j) {
    const int off = 1024 * j + 16 * lane;
    if (EXACT || (vec && off + 16 <= n)) {
      x.v[j][0] = *reinterpret_cast<const u32x4*>(src + off);
      x.v[j][1] = *reinterpret_cast<const u32x4*>(src + off + 8);
    } else {
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int e = off + 2 * i;
        const uint32_t lo = e < n ? src[e] : 0u;
        const uint32_t hi = e + 1 < n ? src[e + 1] : 0u;
        w[i] = lo | (hi << 16);
      }
      x.v[j][0] = (u32x4){w[0], w[1], w[2], w[3]};
      x.v[j][1] = (u32x4){w[4], w[5], w[6], w[7]};
    }
  }
}

// HF RMSNorm of the whole row held by the wave (lane slices of x), in place:
// x := fp16(fp16(x * rsqrt(mean(x^2) + eps)) * w), fp32 mean over n values.
template <int KCH>
__device__ __forceinline__ void x_rmsnorm(XRaw<KCH>& x, const XRaw<KCH>& w, int n, float eps) {
  float ssq = 0.0f;
#pragma unroll
  for (int j = 0; j < KCH; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t q[4] = {x.v[j][h].x, x.v[j][h].y, x.v[j][h].z, x.v[j][h].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = h2f((uint16_t)(q[i] & 0xFFFFu)), b = h2f((uint16_t)(q[i] >> 16));
        ssq = fmaf(a, a, ssq);
        ssq = fmaf(b, b, ssq);
      }
    }
  const float rstd = 1.0f / sqrtf(wave_sum(ssq) / (float)n + eps);
#pragma unroll
  for (int j = 0; j < KCH; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t q[4] = {x.v[j][h].x, x.v[j][h].y, x.v[j][h].z, x.v[j][h].w};
      const uint32_t g[4] = {w.v[j][h].x, w.v[j][h].y, w.v[j][h].z, w.v[j][h].w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint16_t a = f2h(h2f((uint16_t)(q[i] & 0xFFFFu)) * rstd);
        const uint16_t b = f2h(h2f((uint16_t)(q[i] >> 16)) * rstd);
        const uint16_t ya = f2h(h2f(a) * h2f((uint16_t)(g[i] & 0xFFFFu)));
        const uint16_t yb = f2h(h2f(b) * h2f((uint16_t)(g[i] >> 16)));
        o[i] = (uint32_t)ya | ((uint32_t)yb << 16);
      }
      x.v[j][h] = (u32x4){o[0], o[1], o[2], o[3]};
    }
}

template <int KCH>
__device__ __forceinline__ void x_chunks(const XRaw<KCH>& x, XChunk (&xc)[KCH]) {
#pragma unroll
  for (int j = 0; j < KCH; ++j) make_xchunk(x.v[j][0], x.v[j][1], xc[j]);
}

// Keep the scheduler from moving arithmetic above the loads issued so far.
#define LEMOQ_LOADS_ISSUED() __builtin_amdgcn_sched_barrier(0)

// ---------------------------------------------------------------------------
// Routing of one token inside one wave (the arithmetic of
// src/lemoq/kernels/_routing_triton.py:55-80 and moe_static._route,
// src/lemoq/kernels/moe_static.py:276-283): p = exp(z - max) / sum exp(z - max)
// in fp32 over E <= 64*PL values (lane l holds elements l + 64*i), then
// rounds of argmax (ties -> lowest index), optional renormalisation over the
// selected top_k.  Lane k < rounds returns the k-th selection (id, weight).
// `rounds` (1 .. top_k) stops the selection early for a caller that needs
// only the first few ranks; the renormalised weight is exact only when
// rounds == top_k (the sum covers the selected weights).
//
// PL == 1: each round is a DPP wave max of the remaining probabilities, a
// ballot of the lanes equal to it (the lowest such lane wins) and a readlane
// of the winner's weight; no LDS.
// ---------------------------------------------------------------------------
template <int PL>
__device__ __forceinline__ void wave_route(const float (&z)[PL], int E, int top_k, bool norm,
                                           int& my_id, float& my_w, int rounds = -1) {
  const int lane = threadIdx.x & 63;
  if (rounds < 0 || rounds > top_k) rounds = top_k;
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PL; ++i)
    if (lane + 64 * i < E) mx = fmaxf(mx, z[i]);
  mx = wave_max(mx);
  float p[PL];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    p[i] = (lane + 64 * i < E) ? expf(z[i] - mx) : 0.0f;
    sum += p[i];
  }
  sum = wave_sum(sum);
#pragma unroll
  for (int i = 0; i < PL; ++i) p[i] = (lane + 64 * i < E) ? p[i] / sum : -1.0f;
  my_id = 0;
  my_w = 0.0f;
  float wsum = 0.0f;
  if constexpr (PL == 1) {
    float q = p[0];  // remaining candidates; selected lanes drop to -2
    for (int k = 0; k < rounds; ++k) {
      const float m = wave_max(q);
      const int id = (int)__builtin_ctzll(__ballot(q == m));
      const float w = lane_f(p[0], id);
      if (lane == k) {
        my_id = id;
        my_w = w;
      }
      wsum += w;
      if (lane == id) q = -2.0f;
    }
  } else {
    uint32_t taken = 0u;
    for (int k = 0; k < rounds; ++k) {
      float bv = -2.0f;
      int bi = 0x7fffffff;
#pragma unroll
      for (int i = 0; i < PL; ++i) {
        const int idx = lane + 64 * i;
        if (!((taken >> i) & 1u) && idx < E && p[i] > bv) {
          bv = p[i];
          bi = idx;
        }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
      if (lane == k) {
        my_id = bi;
        my_w = bv;
      }
      wsum += bv;
    }
  }
  if (norm) my_w = my_w / wsum;
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
