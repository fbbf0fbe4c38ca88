// Weight formats of the reference's dense dequant operator beyond 8-bit
// symmetric: 8-bit asymmetric (uint8 codes + zero point), 4-bit symmetric
// (int4) and asymmetric (uint4 + zero point), both two codes per byte with the
// low nibble first, and MXFP4 (E2M1 codes, two per byte, one E8M0 byte scale
// per 32 codes).  For each: the decode GEMV (the fused arm of
// dequant_gemm_fused, src/lemoq/kernels/_dequant_triton.py:155-293, kernel
// :313-463), the dequantisation to a dense weight (QuantLinear's separate arm,
// src/lemoq/quant/linear.py:365-395, and mxfp4.dequantize_packed,
// src/lemoq/quant/mxfp4.py:105-122), and the quantisers (rtn.quantize_rtn,
// src/lemoq/quant/rtn.py:38-99 with pack.pack_4bit, src/lemoq/quant/pack.py:21-37;
// mxfp4.quantize_mxfp4, src/lemoq/quant/mxfp4.py:50-102).
//
// GEMV layout (as the w8 GEMV): a 256-thread block is 4 waves, wave w of block
// b owns rows (4b + w) * R ... + R - 1; lane l reads bytes [1024 j + 16 l, +16)
// of chunk j of a packed row (16 codes at 8 bits, 32 at 4 bits), the group
// scale (and zero point) of that slice, and the matching slice of x, all
// issued before any arithmetic.  Codes become exact fp16 values in registers:
//   8-bit: byte permutes against 0x64 (fp16 1024 + u) and one packed subtract;
//   4-bit int: nibble masks, then the same permutes and subtract;
//   E2M1: v_cvt_scalef32_pk_f16_fp4 at scale 1.0 (the values 0 .. 6 and their
//   negatives are exact in fp16; the E8M0 scale is applied in fp32 afterwards).
// v_dot2_f32_f16 forms the products with x exactly in fp32 and accumulates in
// fp32.  Per slice: acc += s * (sum c x - z * sum x), which is the reference's
// sum over k of ((c - z) * s) * x in another fp32 summation order.
#include "qformat.h"

namespace {

using namespace lemoq_qf;

constexpr bool qf_4bit(int f) {
  return f == LEMOQ_QFMT_W4 || f == LEMOQ_QFMT_W4_ASYM || f == LEMOQ_QFMT_MXFP4;
}
constexpr bool qf_asym(int f) { return f == LEMOQ_QFMT_W8_ASYM || f == LEMOQ_QFMT_W4_ASYM; }
constexpr int qf_slice_codes(int f) { return qf_4bit(f) ? 32 : 16; }  // codes per 16-byte slice

// E8M0 byte -> 2^(X - 127) as fp32, exactly as exp2(X - 127.0) in fp32:
// X = 0 is the subnormal 2^-127, X = 255 overflows to +inf.
__device__ __forceinline__ float e8m0_value(uint32_t X) {
  return X == 0u ? __builtin_bit_cast(float, 0x00400000u) : __builtin_bit_cast(float, X << 23);
}

template <int FMT, bool S32>
__device__ __forceinline__ uint32_t load_scale_raw(const void* p, int64_t i) {
  if (FMT == LEMOQ_QFMT_MXFP4) return reinterpret_cast<const uint8_t*>(p)[i];
  if (S32) return reinterpret_cast<const uint32_t*>(p)[i];
  return reinterpret_cast<const uint16_t*>(p)[i];
}

template <int FMT, bool S32>
__device__ __forceinline__ float scale_value(uint32_t raw) {
  if (FMT == LEMOQ_QFMT_MXFP4) return e8m0_value(raw);
  return S32 ? __builtin_bit_cast(float, raw) : h2f((uint16_t)raw);
}

// Unsigned 8-bit codes (0 .. 255) x 16 activations: as dot16_i8 without the
// sign flip (fp16 1024 + u, minus 1024).
__device__ __forceinline__ float dot16_u8(const u32x4 c, const XChunk& xc, float acc) {
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  const f16x2 bias = {(f16)1024.0f, (f16)1024.0f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 clo = as_h2(__builtin_amdgcn_perm(0x64646464u, cw[i], 0x04020400u)) - bias;
    const f16x2 chi = as_h2(__builtin_amdgcn_perm(0x64646464u, cw[i], 0x04030401u)) - bias;
    acc = __builtin_amdgcn_fdot2(clo, xc.a[i], acc, false);
    acc = __builtin_amdgcn_fdot2(chi, xc.b[i], acc, false);
  }
  return acc;
}

// 32 E2M1 codes x 32 activations in natural pairs (xw[m] = x[2m] | x[2m+1] << 16).
// The conversion puts the low nibble of the selected byte in element 0
// (checked on the device for all 256 bytes).
__device__ __forceinline__ float dot32_fp4(const u32x4 c, const uint32_t (&xw)[16], float acc) {
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    acc = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 0), as_h2(xw[4 * d + 0]),
                                 acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 1), as_h2(xw[4 * d + 1]),
                                 acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 2), as_h2(xw[4 * d + 2]),
                                 acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 3), as_h2(xw[4 * d + 3]),
                                 acc, false);
  }
  return acc;
}

struct GemvQArgs {
  const uint16_t* x;
  int64_t x_ld;
  int K;                  // activation width (<= codes per row)
  const uint8_t* codes;   // (N, row_bytes) packed rows
  int row_bytes;
  const void* scale;      // (N, ngroups): fp16 / fp32 / E8M0 bytes
  const void* zero;       // (N, ngroups), same type as scale (asymmetric formats)
  int64_t N;
  int ngroups;
  int group;              // codes per group
  void* y;
  int64_t y_ld;
  int y_f16;
  const uint16_t* residual;  // (M, N) fp16 with ld y_ld, or NULL: y = fp16(fp16(acc) + residual)
  const uint16_t* norm_w;    // (K) fp16 RMSNorm weight of x, or NULL: x as it is
  float eps;
  // RMSNorm instances only: x row *x_row_index of x_rows (M == 1; an index
  // outside reads as a zero row), the raw row copied to x_copy by block 0, and
  // the norm computed once per block through LDS (block_norm) or in every wave
  const int64_t* x_row_index;
  int64_t x_rows;
  uint16_t* x_copy;
  int block_norm;
};

// HF RMSNorm of the row the wave holds (lane slices of NV values per chunk,
// zero past K), in place: x := fp16(fp16(x * rsqrt(mean(x^2) + eps)) * w) with
// an fp32 mean over K values -- the rounding points of rms_norm_fused and of
// the other norm prologues (x_rmsnorm).
template <int KCH, int NV>
__device__ __forceinline__ void xq_rmsnorm(uint32_t (&xw)[KCH][NV / 2], const uint32_t (&nw)[KCH][NV / 2], int K,
                                           float eps) {
  float ssq = 0.0f;
#pragma unroll
  for (int j = 0; j < KCH; ++j)
#pragma unroll
    for (int i = 0; i < NV / 2; ++i) {
      const float a = h2f((uint16_t)(xw[j][i] & 0xFFFFu)), b = h2f((uint16_t)(xw[j][i] >> 16));
      ssq = fmaf(a, a, ssq);
      ssq = fmaf(b, b, ssq);
    }
  const float rstd = 1.0f / sqrtf(wave_sum(ssq) / (float)K + eps);
#pragma unroll
  for (int j = 0; j < KCH; ++j)
#pragma unroll
    for (int i = 0; i < NV / 2; ++i) {
      const uint16_t a = f2h(h2f((uint16_t)(xw[j][i] & 0xFFFFu)) * rstd);
      const uint16_t b = f2h(h2f((uint16_t)(xw[j][i] >> 16)) * rstd);
      const uint16_t ya = f2h(h2f(a) * h2f((uint16_t)(nw[j][i] & 0xFFFFu)));
      const uint16_t yb = f2h(h2f(b) * h2f((uint16_t)(nw[j][i] >> 16)));
      xw[j][i] = (uint32_t)ya | ((uint32_t)yb << 16);
    }
}

// The wave's R rows x KCH chunks of codes, their scales (and zero points).
template <int FMT, int KCH, int R, bool S32>
__device__ __forceinline__ uint32_t gemv_q_issue(const GemvQArgs& a, int64_t row0, int lane, u32x4 (&c)[R][KCH],
                                                 uint32_t (&sraw)[R][KCH], uint32_t (&zraw)[R][KCH]) {
  constexpr int NV = qf_slice_codes(FMT);
  constexpr bool ASYM = qf_asym(FMT);
  uint32_t ok = 0u;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = row0 + r;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int off = 1024 * j + 16 * lane;
      const bool in = row < a.N && off < a.row_bytes;
      const int64_t rr = in ? row : 0;
      const int oo = in ? off : 0;
      c[r][j] = load_stream16(reinterpret_cast<const int8_t*>(a.codes) + rr * a.row_bytes + oo);
      const int64_t si = rr * a.ngroups + (oo / 16) * NV / a.group;
      sraw[r][j] = load_scale_raw<FMT, S32>(a.scale, si);
      zraw[r][j] = ASYM ? load_scale_raw<FMT, S32>(a.zero, si) : 0u;
      ok |= (in ? 1u : 0u) << (r * KCH + j);
    }
  }
  return ok;
}

template <int FMT, int KCH, int R, bool S32, bool NORM = false>
__global__ __launch_bounds__(256) void gemv_q_kernel(const GemvQArgs a) {
  constexpr int NV = qf_slice_codes(FMT);
  constexpr int CPC = 64 * NV;  // codes per 1 KB chunk
  constexpr bool ASYM = qf_asym(FMT);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m = blockIdx.y;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * R;

  u32x4 c[R][KCH];
  uint32_t sraw[R][KCH], zraw[R][KCH];
  uint32_t ok = 0u;
  uint32_t xw[KCH][NV / 2];
  if constexpr (!NORM) {
    ok = gemv_q_issue<FMT, KCH, R, S32>(a, row0, lane, c, sraw, zraw);
    const uint16_t* xr = a.x + m * a.x_ld;
    const bool vec = ((reinterpret_cast<uintptr_t>(xr) & 15u) == 0) && ((a.K & 7) == 0);
#pragma unroll
    for (int j = 0; j < KCH; ++j) xq_load<NV>(xw[j], xr, a.K, j * CPC + lane * NV, vec);
    LEMOQ_LOADS_ISSUED();
  } else {
    // RMSNorm prologue.  The row and the norm weight are loaded first (the
    // memory counter retires in order, so the norm waits only for them while
    // the weight codes stream in).  Rows that fill the chunks exactly, K a
    // multiple of 2048: once per block (8 values a thread, an LDS reduction,
    // the normalised row in LDS); otherwise in every wave from its slices.
    bool x_ok = true;
    const uint16_t* xr = a.x + m * a.x_ld;
    if (a.x_row_index) {
      const int64_t r = a.x_row_index[0];
      x_ok = r >= 0 && r < a.x_rows;  // an index outside the table reads as a zero row
      xr = a.x + (x_ok ? r : 0) * a.x_ld;
    }
    constexpr int BNV = (KCH * CPC) % 2048 == 0 ? (KCH * CPC) / 2048 : 1;  // u32x4 a thread, block form
    constexpr bool kBlockForm = (KCH * CPC) % 2048 == 0;
    if (kBlockForm && a.block_norm) {
      __shared__ __align__(16) uint16_t xs[KCH * CPC];
      __shared__ float red[4];
      u32x4 rv[BNV], wv[BNV];
#pragma unroll
      for (int i = 0; i < BNV; ++i) {
        const int off = (i * 256 + threadIdx.x) * 8;
        rv[i] = *reinterpret_cast<const u32x4*>(xr + off);
        wv[i] = *reinterpret_cast<const u32x4*>(a.norm_w + off);
      }
      ok = gemv_q_issue<FMT, KCH, R, S32>(a, row0, lane, c, sraw, zraw);
      LEMOQ_LOADS_ISSUED();
      float ssq = 0.0f;
#pragma unroll
      for (int i = 0; i < BNV; ++i) {
        if (!x_ok) rv[i] = (u32x4){0u, 0u, 0u, 0u};
        const uint32_t q[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float x0 = h2f((uint16_t)(q[k] & 0xFFFFu)), x1 = h2f((uint16_t)(q[k] >> 16));
          ssq = fmaf(x0, x0, ssq);
          ssq = fmaf(x1, x1, ssq);
        }
        if (a.x_copy && blockIdx.x == 0 && m == 0)
          *reinterpret_cast<u32x4*>(a.x_copy + (i * 256 + threadIdx.x) * 8) = rv[i];
      }
      ssq = wave_sum(ssq);
      if (lane == 0) red[wave] = ssq;
      __syncthreads();
      const float rstd = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)a.K + a.eps);
#pragma unroll
      for (int i = 0; i < BNV; ++i) {
        const uint32_t q[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w};
        const uint32_t g[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint16_t n0 = f2h(h2f((uint16_t)(q[k] & 0xFFFFu)) * rstd);
          const uint16_t n1 = f2h(h2f((uint16_t)(q[k] >> 16)) * rstd);
          const uint16_t y0 = f2h(h2f(n0) * h2f((uint16_t)(g[k] & 0xFFFFu)));
          const uint16_t y1 = f2h(h2f(n1) * h2f((uint16_t)(g[k] >> 16)));
          o[k] = (uint32_t)y0 | ((uint32_t)y1 << 16);
        }
        *reinterpret_cast<u32x4*>(xs + (i * 256 + threadIdx.x) * 8) = (u32x4){o[0], o[1], o[2], o[3]};
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < KCH; ++j)
#pragma unroll
        for (int q = 0; q < NV / 8; ++q) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(xs + j * CPC + lane * NV + 8 * q);
          xw[j][4 * q + 0] = v.x;
          xw[j][4 * q + 1] = v.y;
          xw[j][4 * q + 2] = v.z;
          xw[j][4 * q + 3] = v.w;
        }
    } else {
      const bool vec = ((reinterpret_cast<uintptr_t>(xr) & 15u) == 0) && ((a.K & 7) == 0);
      const bool vw = ((reinterpret_cast<uintptr_t>(a.norm_w) & 15u) == 0) && ((a.K & 7) == 0);
      uint32_t nw[KCH][NV / 2];
#pragma unroll
      for (int j = 0; j < KCH; ++j) {
        xq_load<NV>(xw[j], xr, a.K, j * CPC + lane * NV, vec);
        xq_load<NV>(nw[j], a.norm_w, a.K, j * CPC + lane * NV, vw);
      }
      ok = gemv_q_issue<FMT, KCH, R, S32>(a, row0, lane, c, sraw, zraw);
      LEMOQ_LOADS_ISSUED();
      if (!x_ok) {
#pragma unroll
        for (int j = 0; j < KCH; ++j)
#pragma unroll
          for (int i = 0; i < NV / 2; ++i) xw[j][i] = 0u;
      }
      xq_rmsnorm<KCH, NV>(xw, nw, a.K, a.eps);
    }
  }

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int j = 0; j < KCH; ++j) {
    float xs = 0.0f;  // sum of the slice's activations (zero-point term)
    if (ASYM) {
      const f16x2 one = {(f16)1.0f, (f16)1.0f};
#pragma unroll
      for (int i = 0; i < NV / 2; ++i) xs = __builtin_amdgcn_fdot2(as_h2(xw[j][i]), one, xs, false);
    }
    XChunk x0, x1;
    if constexpr (FMT != LEMOQ_QFMT_MXFP4) {
      xchunk_of(&xw[j][0], x0);
      if constexpr (NV == 32) xchunk_of(&xw[j][8], x1);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float d;
      if constexpr (FMT == LEMOQ_QFMT_W8) d = dot16_i8(c[r][j], x0, 0.0f);
      else if constexpr (FMT == LEMOQ_QFMT_W8_ASYM) d = dot16_u8(c[r][j], x0, 0.0f);
      else if constexpr (FMT == LEMOQ_QFMT_W4) d = dot32_i4<true>(c[r][j], x0, x1, 0.0f);
      else if constexpr (FMT == LEMOQ_QFMT_W4_ASYM) d = dot32_i4<false>(c[r][j], x0, x1, 0.0f);
      else d = dot32_fp4(c[r][j], xw[j], 0.0f);
      if (ASYM) d = fmaf(-scale_value<FMT, S32>(zraw[r][j]), xs, d);
      const bool use = (ok >> (r * KCH + j)) & 1u;
      acc[r] = use ? fmaf(scale_value<FMT, S32>(sraw[r][j]), d, acc[r]) : acc[r];
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
  if (lane < R) {
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) v = acc[r];
    const int64_t n = row0 + lane;
    if (n < a.N) {
      if (a.residual)  // the fp16 residual add after the projection (one rounding of the fp16 sum)
        reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + n] = hadd_round(h2f(f2h(v)), a.residual[m * a.y_ld + n]);
      else if (a.y_f16)
        reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + n] = f2h(v);
      else
        reinterpret_cast<float*>(a.y)[m * a.y_ld + n] = v;
    }
  }
}

#ifndef LEMOQ_GEMVQ_ROWS
#define LEMOQ_GEMVQ_ROWS 2  // rows per wave, as the w8 GEMV
#endif
constexpr int kGemvQRows = LEMOQ_GEMVQ_ROWS;

template <int FMT, bool S32, bool NORM>
int launch_gemv_q(int kch, dim3 grid, hipStream_t st, const GemvQArgs& a) {
  switch (kch) {
    case 1: hipLaunchKernelGGL((gemv_q_kernel<FMT, 1, kGemvQRows, S32, NORM>), grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL((gemv_q_kernel<FMT, 2, kGemvQRows, S32, NORM>), grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL((gemv_q_kernel<FMT, 4, kGemvQRows, S32, NORM>), grid, dim3(256), 0, st, a); break;
    case 8:
      if constexpr (!qf_4bit(FMT)) {
        hipLaunchKernelGGL((gemv_q_kernel<FMT, 8, kGemvQRows, S32, NORM>), grid, dim3(256), 0, st, a);
        break;
      }
      return LEMOQ_ERR_UNSUPPORTED;
    default: return LEMOQ_ERR_UNSUPPORTED;
  }
  LEMOQ_CHECK_LAUNCH();
}

// The RMSNorm prologue is instantiated for fp16 (or E8M0) scales only.
template <int FMT>
int launch_gemv_q_fmt(bool s32, int kch, dim3 grid, hipStream_t st, const GemvQArgs& a) {
  if (a.norm_w) return s32 ? LEMOQ_ERR_UNSUPPORTED : launch_gemv_q<FMT, false, true>(kch, grid, st, a);
  if constexpr (FMT == LEMOQ_QFMT_MXFP4) return launch_gemv_q<FMT, false, false>(kch, grid, st, a);
  else
    return s32 ? launch_gemv_q<FMT, true, false>(kch, grid, st, a) : launch_gemv_q<FMT, false, false>(kch, grid, st, a);
}

// ---------------------------------------------------------------------------
// The same GEMV on fp32 activations (the reference's dequant_gemm_fused takes
// x in fp16 or fp32, src/lemoq/kernels/_dequant_triton.py:252-253).  fp32 x
// cannot enter v_dot2_f32_f16, so each code becomes an fp32 value (exact: 8-bit
// and 4-bit integers, E2M1's 0 .. 6) and is multiplied with x in fp32 FMAs;
// per slice acc += s * (sum c x - z * sum x) as above.  The load order is the
// fp16 kernel's: every code slice, scale and x slice before any arithmetic.
// ---------------------------------------------------------------------------
template <int FMT>
__device__ __forceinline__ void codes_to_f32(const u32x4 c, float (&v)[qf_slice_codes(FMT)]) {
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  if constexpr (FMT == LEMOQ_QFMT_MXFP4) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const f16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 0);
      const f16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 1);
      const f16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 2);
      const f16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 3);
      v[8 * d + 0] = (float)p0[0];
      v[8 * d + 1] = (float)p0[1];
      v[8 * d + 2] = (float)p1[0];
      v[8 * d + 3] = (float)p1[1];
      v[8 * d + 4] = (float)p2[0];
      v[8 * d + 5] = (float)p2[1];
      v[8 * d + 6] = (float)p3[0];
      v[8 * d + 7] = (float)p3[1];
    }
  } else if constexpr (qf_4bit(FMT)) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const uint32_t nib = (cw[i >> 3] >> (4 * (i & 7))) & 0xFu;
      v[i] = FMT == LEMOQ_QFMT_W4 ? (float)((int)(nib ^ 8u) - 8) : (float)nib;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t b = (cw[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      v[i] = FMT == LEMOQ_QFMT_W8 ? (float)(int)(int8_t)b : (float)b;
    }
  }
}

struct GemvQ32Args {
  const float* x;
  int64_t x_ld;
  int K;
  const uint8_t* codes;
  int row_bytes;
  const void* scale;
  const void* zero;
  int64_t N;
  int ngroups;
  int group;
  void* y;
  int64_t y_ld;
  int y_f16;
};

template <int FMT, int KCH, int R, bool S32>
__global__ __launch_bounds__(256) void gemv_q_x32_kernel(const GemvQ32Args a) {
  constexpr int NV = qf_slice_codes(FMT);
  constexpr int CPC = 64 * NV;
  constexpr bool ASYM = qf_asym(FMT);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m = blockIdx.y;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * R;

  u32x4 c[R][KCH];
  uint32_t sraw[R][KCH], zraw[R][KCH];
  uint32_t ok = 0u;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = row0 + r;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int off = 1024 * j + 16 * lane;
      const bool in = row < a.N && off < a.row_bytes;
      const int64_t rr = in ? row : 0;
      const int oo = in ? off : 0;
      c[r][j] = load_stream16(reinterpret_cast<const int8_t*>(a.codes) + rr * a.row_bytes + oo);
      const int64_t si = rr * a.ngroups + (oo / 16) * NV / a.group;
      sraw[r][j] = load_scale_raw<FMT, S32>(a.scale, si);
      zraw[r][j] = ASYM ? load_scale_raw<FMT, S32>(a.zero, si) : 0u;
      ok |= (in ? 1u : 0u) << (r * KCH + j);
    }
  }
  // x: the lane's NV consecutive fp32 values of each chunk, zero past K
  const float* xr = a.x + m * a.x_ld;
  const bool vec = ((reinterpret_cast<uintptr_t>(xr) & 15u) == 0) && ((a.K & 3) == 0);
  float xv[KCH][NV];
#pragma unroll
  for (int j = 0; j < KCH; ++j) {
    const int k0 = j * CPC + lane * NV;
    if (vec && k0 + NV <= a.K) {
#pragma unroll
      for (int q = 0; q < NV / 4; ++q) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(xr + k0 + 4 * q);
        xv[j][4 * q + 0] = as_f32(w.x);
        xv[j][4 * q + 1] = as_f32(w.y);
        xv[j][4 * q + 2] = as_f32(w.z);
        xv[j][4 * q + 3] = as_f32(w.w);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NV; ++i) xv[j][i] = k0 + i < a.K ? xr[k0 + i] : 0.0f;
    }
  }
  LEMOQ_LOADS_ISSUED();

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int j = 0; j < KCH; ++j) {
    float xs = 0.0f;
    if (ASYM) {
#pragma unroll
      for (int i = 0; i < NV; ++i) xs += xv[j][i];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float cv[NV];
      codes_to_f32<FMT>(c[r][j], cv);
      float d = 0.0f;
#pragma unroll
      for (int i = 0; i < NV; ++i) d = fmaf(cv[i], xv[j][i], d);
      if (ASYM) d = fmaf(-scale_value<FMT, S32>(zraw[r][j]), xs, d);
      const bool use = (ok >> (r * KCH + j)) & 1u;
      acc[r] = use ? fmaf(scale_value<FMT, S32>(sraw[r][j]), d, acc[r]) : acc[r];
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
  if (lane < R) {
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) v = acc[r];
    const int64_t n = row0 + lane;
    if (n < a.N) {
      if (a.y_f16)
        reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + n] = f2h(v);
      else
        reinterpret_cast<float*>(a.y)[m * a.y_ld + n] = v;
    }
  }
}

template <int FMT, bool S32>
int launch_gemv_q_x32(int kch, dim3 grid, hipStream_t st, const GemvQ32Args& a) {
  switch (kch) {
    case 1: hipLaunchKernelGGL((gemv_q_x32_kernel<FMT, 1, kGemvQRows, S32>), grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL((gemv_q_x32_kernel<FMT, 2, kGemvQRows, S32>), grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL((gemv_q_x32_kernel<FMT, 4, kGemvQRows, S32>), grid, dim3(256), 0, st, a); break;
    case 8:
      if constexpr (!qf_4bit(FMT)) {
        hipLaunchKernelGGL((gemv_q_x32_kernel<FMT, 8, kGemvQRows, S32>), grid, dim3(256), 0, st, a);
        break;
      }
      return LEMOQ_ERR_UNSUPPORTED;
    default: return LEMOQ_ERR_UNSUPPORTED;
  }
  LEMOQ_CHECK_LAUNCH();
}

template <int FMT>
int launch_gemv_q_x32_fmt(bool s32, int kch, dim3 grid, hipStream_t st, const GemvQ32Args& a) {
  if constexpr (FMT == LEMOQ_QFMT_MXFP4) return launch_gemv_q_x32<FMT, false>(kch, grid, st, a);
  else return s32 ? launch_gemv_q_x32<FMT, true>(kch, grid, st, a) : launch_gemv_q_x32<FMT, false>(kch, grid, st, a);
}

// Shape rules shared by the GEMV and the dequantisation.  Returns 0 or a
// LEMOQ_ERR_* status.
int check_format(int fmt, const void* qweight, const void* scale, const void* zero, int scale_is_f32,
                 int64_t N, int64_t padded_k, int64_t group) {
  if (fmt < LEMOQ_QFMT_W8 || fmt > LEMOQ_QFMT_MXFP4) return LEMOQ_ERR_UNSUPPORTED;
  if (!qweight || !scale) return LEMOQ_ERR_NULL;
  const bool asym = fmt == LEMOQ_QFMT_W8_ASYM || fmt == LEMOQ_QFMT_W4_ASYM;
  if (asym && !zero) return LEMOQ_ERR_NULL;
  if (fmt == LEMOQ_QFMT_MXFP4 && (group != 32 || scale_is_f32 || zero)) return LEMOQ_ERR_UNSUPPORTED;
  if (N <= 0 || N > 0x7fffffffLL || padded_k <= 0 || group <= 0) return LEMOQ_ERR_SHAPE;
  const int nv = (fmt == LEMOQ_QFMT_W8 || fmt == LEMOQ_QFMT_W8_ASYM) ? 16 : 32;
  if (group % nv != 0 || padded_k % group != 0 || padded_k > 8192) return LEMOQ_ERR_UNSUPPORTED;
  if (!lemoq_aligned16(qweight)) return LEMOQ_ERR_ALIGN;
  return LEMOQ_OK;
}

// ---------------------------------------------------------------------------
// Dequantisation to a dense weight, one thread per 16-byte slice of codes:
// w = c * s (symmetric), (c - z) * s (asymmetric), e2m1(c) * 2^(X - 127)
// (MXFP4), each in fp32 as the reference's separate arm computes it, then
// stored as fp32 or rounded once to fp16 (`.to(dtype)`).  Columns at or past
// k_out are not written.
// ---------------------------------------------------------------------------
struct DequantQArgs {
  const uint8_t* codes;
  int row_bytes;
  const void* scale;
  const void* zero;
  int64_t N;
  int ngroups;
  int group;
  void* w;
  int64_t ld;
  int k_out;
};

template <int FMT, bool S32, bool OUT32>
__global__ __launch_bounds__(256) void dequant_q_kernel(const DequantQArgs a) {
  constexpr int NV = qf_slice_codes(FMT);
  const int64_t spr = a.row_bytes / 16;  // slices per row
  const int64_t sl = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (sl >= a.N * spr) return;
  const int64_t row = sl / spr;
  const int k0 = (int)(sl - row * spr) * NV;
  if (k0 >= a.k_out) return;
  const u32x4 c = *reinterpret_cast<const u32x4*>(a.codes + row * a.row_bytes + (k0 / NV) * 16);
  const int64_t si = row * a.ngroups + k0 / a.group;
  const float s = scale_value<FMT, S32>(load_scale_raw<FMT, S32>(a.scale, si));
  const float z = qf_asym(FMT) ? scale_value<FMT, S32>(load_scale_raw<FMT, S32>(a.zero, si)) : 0.0f;
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float code;
    if (NV == 16) {
      const uint32_t b = (cw[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      code = FMT == LEMOQ_QFMT_W8 ? (float)(int)(int8_t)b : (float)b;
    } else {
      const uint32_t nib = (cw[i >> 3] >> (4 * (i & 7))) & 0xFu;
      if (FMT == LEMOQ_QFMT_W4) code = (float)((int)(nib ^ 8u) - 8);
      else if (FMT == LEMOQ_QFMT_W4_ASYM) code = (float)nib;
      else code = 0.0f;  // MXFP4 below
    }
    v[i] = code;
  }
  if (FMT == LEMOQ_QFMT_MXFP4) {
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        f16x2 p;
        switch (b) {
          case 0: p = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 0); break;
          case 1: p = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 1); break;
          case 2: p = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 2); break;
          default: p = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(cw[d], 1.0f, 3); break;
        }
        v[8 * d + 2 * b] = (float)p[0];
        v[8 * d + 2 * b + 1] = (float)p[1];
      }
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = qf_asym(FMT) ? (v[i] - z) * s : v[i] * s;
  if (OUT32) {
    float* dst = reinterpret_cast<float*>(a.w) + row * a.ld + k0;
    for (int i = 0; i < NV && k0 + i < a.k_out; ++i) dst[i] = v[i];
  } else {
    uint16_t* dst = reinterpret_cast<uint16_t*>(a.w) + row * a.ld + k0;
    const bool vec = k0 + NV <= a.k_out && ((reinterpret_cast<uintptr_t>(dst) & 15u) == 0);
    if (vec) {
#pragma unroll
      for (int q = 0; q < NV / 8; ++q) {
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[i] = (uint32_t)f2h(v[8 * q + 2 * i]) | ((uint32_t)f2h(v[8 * q + 2 * i + 1]) << 16);
        *reinterpret_cast<u32x4*>(dst + 8 * q) = (u32x4){o[0], o[1], o[2], o[3]};
      }
    } else {
      for (int i = 0; i < NV && k0 + i < a.k_out; ++i) dst[i] = f2h(v[i]);
    }
  }
}

template <int FMT, bool S32>
int launch_dequant_q2(bool out32, dim3 grid, hipStream_t st, const DequantQArgs& a) {
  if (out32)
    hipLaunchKernelGGL((dequant_q_kernel<FMT, S32, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((dequant_q_kernel<FMT, S32, false>), grid, dim3(256), 0, st, a);
  LEMOQ_CHECK_LAUNCH();
}

template <int FMT>
int launch_dequant_q(bool s32, bool out32, dim3 grid, hipStream_t st, const DequantQArgs& a) {
  if constexpr (FMT == LEMOQ_QFMT_MXFP4) return launch_dequant_q2<FMT, false>(out32, grid, st, a);
  else return s32 ? launch_dequant_q2<FMT, true>(out32, grid, st, a) : launch_dequant_q2<FMT, false>(out32, grid, st, a);
}

// ---------------------------------------------------------------------------
// Per-group RTN at 4 or 8 bits, symmetric or asymmetric, one wave per
// (row, group) (src/lemoq/quant/rtn.py:58-87):
//   symmetric:  s = absmax / qmax (1 when absmax == 0), c = clamp(rint(w / s),
//               -(qmax + 1), qmax), zero 0;
//   asymmetric: over the real columns only (the zero padding of the last
//               group is left out of min / max), gmax / gmin (0 when not
//               finite), s = (gmax - gmin) / qmax (1 when the range is 0),
//               z = rint(-gmin / s), c = clamp(rint(w / s) + z, 0, qmax).
// All in fp32 with IEEE division and round-half-even.  4-bit codes are packed
// two per byte, the even column in the low nibble (pack.pack_4bit).
// ---------------------------------------------------------------------------
template <int BITS, bool SYM>
__global__ __launch_bounds__(256) void rtn_q_kernel(const float* __restrict__ w, int64_t rows, int64_t cols,
                                                    int64_t group, int64_t ngroups, uint8_t* __restrict__ codes,
                                                    int64_t code_ld, uint16_t* __restrict__ s16,
                                                    float* __restrict__ s32, uint16_t* __restrict__ z16,
                                                    float* __restrict__ z32) {
  constexpr float QMAX = SYM ? (float)((1 << (BITS - 1)) - 1) : (float)((1 << BITS) - 1);
  const int lane = threadIdx.x & 63;
  const int64_t gid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gid >= rows * ngroups) return;
  const int64_t row = gid / ngroups;
  const int64_t k0 = (gid - row * ngroups) * group;
  const float* wr = w + row * cols;
  float s, z = 0.0f;
  if (SYM) {
    float amax = 0.0f;
    for (int64_t i = lane; i < group; i += 64) {
      const int64_t k = k0 + i;
      amax = fmaxf(amax, fabsf(k < cols ? wr[k] : 0.0f));
    }
    amax = wave_max(amax);
    s = amax > 0.0f ? amax / QMAX : 1.0f;
  } else {
    float gmax = -INFINITY, gmin = INFINITY;
    for (int64_t i = lane; i < group; i += 64) {
      const int64_t k = k0 + i;
      if (k < cols) {
        gmax = fmaxf(gmax, wr[k]);
        gmin = fminf(gmin, wr[k]);
      }
    }
    gmax = wave_max(gmax);
    gmin = -wave_max(-gmin);
    if (!__builtin_isfinite(gmax)) gmax = 0.0f;
    if (!__builtin_isfinite(gmin)) gmin = 0.0f;
    const float rng = gmax - gmin;
    s = rng > 0.0f ? rng / QMAX : 1.0f;
    z = rintf(-gmin / s);
  }
  const float lo = SYM ? -(QMAX + 1.0f) : 0.0f;
  if (BITS == 8) {
    for (int64_t i = lane; i < group; i += 64) {
      const int64_t k = k0 + i;
      float q = rintf((k < cols ? wr[k] : 0.0f) / s);
      if (!SYM) q = q + z;
      q = fminf(fmaxf(q, lo), QMAX);
      codes[row * code_ld + k] = SYM ? (uint8_t)(int8_t)(int)q : (uint8_t)(int)q;
    }
  } else {
    for (int64_t i = 2 * lane; i < group; i += 128) {  // a pair of columns per byte
      const int64_t k = k0 + i;
      float q0 = rintf((k < cols ? wr[k] : 0.0f) / s);
      float q1 = rintf((k + 1 < cols ? wr[k + 1] : 0.0f) / s);
      if (!SYM) {
        q0 = q0 + z;
        q1 = q1 + z;
      }
      q0 = fminf(fmaxf(q0, lo), QMAX);
      q1 = fminf(fmaxf(q1, lo), QMAX);
      const uint32_t b = ((uint32_t)(int)q0 & 0xFu) | (((uint32_t)(int)q1 & 0xFu) << 4);
      codes[row * code_ld + k / 2] = (uint8_t)b;
    }
  }
  if (lane == 0) {
    if (s16) s16[gid] = f2h(s);
    if (s32) s32[gid] = s;
    if (z16) z16[gid] = f2h(z);
    if (z32) z32[gid] = z;
  }
}

// ---------------------------------------------------------------------------
// MXFP4 quantiser (src/lemoq/quant/mxfp4.py:50-102), two blocks of 32 columns
// per wave (lanes 0-31 and 32-63), columns past `cols` read as 0:
//   X = clamp(floor(log2(amax)) - 2, -127, 127), X = -127 for an all-zero
//   block; the scale byte is X + 127;
//   v = w / 2^X (exact: a power-of-two scaling), m = min(|v|, 6);
//   the magnitude code is the first index of the smallest |m - M[i]| over
//   M = {0, 0.5, 1, 1.5, 2, 3, 4, 6} (ties go to the smaller magnitude);
//   code = (v < 0) << 3 | index; two codes per byte, even column low.
// log2 follows torch's fp32 log2 (the correctly rounded value, which is what
// the floor sees: amax one ulp below 2^k gives k, not k - 1): the double
// log2 rounded to fp32.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mxfp4_quant_kernel(const float* __restrict__ w, int64_t rows, int64_t cols,
                                                          int64_t nblk, uint8_t* __restrict__ codes,
                                                          uint8_t* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int64_t blk = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 2 + (lane >> 5);
  const bool live = blk < rows * nblk;
  const int64_t b = live ? blk : 0;
  const int64_t row = b / nblk, bi = b - row * nblk;
  const int64_t col = bi * 32 + (lane & 31);
  const float v = (live && col < cols) ? w[row * cols + col] : 0.0f;
  const float amax = group_max<32>(fabsf(v));
  float X = -127.0f;
  if (amax > 0.0f) X = fminf(fmaxf(floorf((float)log2((double)amax)) - 2.0f, -127.0f), 127.0f);
  const float nv = ldexpf(v, -(int)X);
  const float mag = fminf(fabsf(nv), 6.0f);
  const float M[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  int idx = 0;
  float best = fabsf(mag - M[0]);
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    const float d = fabsf(mag - M[i]);
    if (d < best) {
      best = d;
      idx = i;
    }
  }
  const uint32_t code = (nv < 0.0f ? 8u : 0u) | (uint32_t)idx;
  const uint32_t hi = (uint32_t)__shfl_xor((int)code, 1, LEMOQ_WAVE);
  if (live && (lane & 1) == 0) codes[row * nblk * 16 + (bi * 32 + (lane & 31)) / 2] = (uint8_t)(code | (hi << 4));
  if (live && (lane & 31) == 0) scales[b] = (uint8_t)(int)(X + 127.0f);
}

// ---------------------------------------------------------------------------
// Per-token symmetric int8 fake quantisation of activations (the w8a8
// scheme's QuantLinear._fake_quant_activation, src/lemoq/quant/linear.py:398-414),
// one wave per row: fp32 absmax, s = absmax / 127 (1 when 0),
// q = clamp(rint(x / s), -128, 127), y = fp16(q * s) (fp32 product, one rounding).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fake_quant_rows_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                              int D, uint16_t* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const uint16_t* xr = x + r * D;
  uint16_t* yr = y + r * D;
  float amax = 0.0f;
  for (int d = lane; d < D; d += 64) amax = fmaxf(amax, fabsf(h2f(xr[d])));
  amax = wave_max(amax);
  const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
  for (int d = lane; d < D; d += 64) {
    const float q = fminf(fmaxf(rintf(h2f(xr[d]) / s), -128.0f), 127.0f);
    yr[d] = f2h(q * s);
  }
}

}  // namespace

extern "C" int lemoq_fake_quant_rows(const uint16_t* x, int64_t rows, int64_t D, uint16_t* y, void* stream) {
  if (!x || !y) return LEMOQ_ERR_NULL;
  if (rows < 0 || D <= 0 || D > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  if (rows == 0) return LEMOQ_OK;
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(fake_quant_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, lemoq_stream(stream), x, rows,
                     (int)D, y);
  LEMOQ_CHECK_LAUNCH();
}

namespace {

struct NormOpts {
  const uint16_t* norm_w;
  float eps;
  const int64_t* x_row_index;
  int64_t x_rows;
  uint16_t* x_copy;
};

int gemv_q_common(const uint16_t* x, int64_t M, int64_t K, const void* qweight, int fmt, const void* scale,
                  const void* zero, int scale_is_f32, int64_t N, int64_t padded_k, int64_t group, void* y,
                  int y_is_f16, const uint16_t* residual, void* stream, const NormOpts* norm = nullptr);

}  // namespace

extern "C" int lemoq_gemv_q(const uint16_t* x, int64_t M, int64_t K, const void* qweight, int fmt,
                            const void* scale, const void* zero, int scale_is_f32, int64_t N,
                            int64_t padded_k, int64_t group, void* y, int y_is_f16, void* stream) {
  return gemv_q_common(x, M, K, qweight, fmt, scale, zero, scale_is_f32, N, padded_k, group, y, y_is_f16,
                       nullptr, stream);
}

extern "C" int lemoq_gemv_q_rmsnorm(const uint16_t* x, const int64_t* x_row_index, int64_t x_rows, int64_t M,
                                    int64_t K, const uint16_t* norm_w, float eps, uint16_t* x_copy,
                                    const void* qweight, int fmt, const void* scale, const void* zero,
                                    int scale_is_f32, int64_t N, int64_t padded_k, int64_t group, void* y,
                                    int y_is_f16, void* stream) {
  if (!norm_w || !x) return LEMOQ_ERR_NULL;
  if (!(eps >= 0.0f)) return LEMOQ_ERR_SHAPE;  // negative or NaN eps
  if (scale_is_f32) return LEMOQ_ERR_UNSUPPORTED;  // the norm prologue takes fp16 (or E8M0) scales
  if (x_row_index && (M != 1 || x_rows <= 0)) return LEMOQ_ERR_SHAPE;
  NormOpts o;
  o.norm_w = norm_w;
  o.eps = eps;
  o.x_row_index = x_row_index;
  o.x_rows = x_row_index ? x_rows : 0;
  o.x_copy = x_copy;
  return gemv_q_common(x, M, K, qweight, fmt, scale, zero, scale_is_f32, N, padded_k, group, y, y_is_f16,
                       nullptr, stream, &o);
}

extern "C" int lemoq_gemv_q_residual(const uint16_t* x, int64_t M, int64_t K, const void* qweight, int fmt,
                                     const void* scale, const void* zero, int scale_is_f32, int64_t N,
                                     int64_t padded_k, int64_t group, const uint16_t* residual, uint16_t* y,
                                     void* stream) {
  if (!residual || !y) return LEMOQ_ERR_NULL;
  // residual is y itself (each element read, then written, by one lane) or apart from it
  if (M > 0 && N > 0 && residual != y) {
    const char* r = reinterpret_cast<const char*>(residual);
    const char* o = reinterpret_cast<const char*>(y);
    const int64_t nb = M * N * 2;
    if (r < o + nb && o < r + nb) return LEMOQ_ERR_SHAPE;
  }
  return gemv_q_common(x, M, K, qweight, fmt, scale, zero, scale_is_f32, N, padded_k, group, y, 1, residual,
                       stream);
}

namespace {

int gemv_q_common(const uint16_t* x, int64_t M, int64_t K, const void* qweight, int fmt, const void* scale,
                  const void* zero, int scale_is_f32, int64_t N, int64_t padded_k, int64_t group, void* y,
                  int y_is_f16, const uint16_t* residual, void* stream, const NormOpts* norm) {
  if (!x || !y) return LEMOQ_ERR_NULL;
  const int rc = check_format(fmt, qweight, scale, zero, scale_is_f32, N, padded_k, group);
  if (rc) return rc;
  if (M <= 0 || M > 65535 || K <= 0 || K > padded_k) return LEMOQ_ERR_SHAPE;
  GemvQArgs a;
  a.x = x;
  a.x_ld = K;
  a.K = (int)K;
  a.codes = reinterpret_cast<const uint8_t*>(qweight);
  const bool four = qf_4bit(fmt);
  a.row_bytes = (int)(four ? padded_k / 2 : padded_k);
  a.scale = scale;
  a.zero = zero;
  a.N = N;
  a.ngroups = (int)(padded_k / group);
  a.group = (int)group;
  a.y = y;
  a.y_ld = N;
  a.y_f16 = y_is_f16 ? 1 : 0;
  a.residual = residual;
  a.norm_w = norm ? norm->norm_w : nullptr;
  a.eps = norm ? norm->eps : 0.0f;
  a.x_row_index = norm ? norm->x_row_index : nullptr;
  a.x_rows = norm ? norm->x_rows : 0;
  a.x_copy = norm ? norm->x_copy : nullptr;
  const int64_t chunks = (a.row_bytes + 1023) / 1024;
  const int kch = chunks <= 1 ? 1 : (chunks <= 2 ? 2 : (chunks <= 4 ? 4 : 8));
  // the block form of the norm: rows that fill the kernel's chunks exactly, a
  // multiple of 2048 values, 16-byte aligned rows (x_copy needs it)
  const int64_t cpc = 64 * (qf_4bit(fmt) ? 32 : 16);
  a.block_norm = norm && K == kch * cpc && K % 2048 == 0 && lemoq_aligned16(x) && lemoq_aligned16(a.norm_w) &&
                 (!a.x_copy || lemoq_aligned16(a.x_copy));
  if (norm && a.x_copy && !a.block_norm) return LEMOQ_ERR_UNSUPPORTED;
  const int64_t blocks = (N + 4 * kGemvQRows - 1) / (4 * kGemvQRows);
  const dim3 grid((unsigned)blocks, (unsigned)M);
  hipStream_t st = lemoq_stream(stream);
  const bool s32 = scale_is_f32 != 0;
  switch (fmt) {
    case LEMOQ_QFMT_W8: return launch_gemv_q_fmt<LEMOQ_QFMT_W8>(s32, kch, grid, st, a);
    case LEMOQ_QFMT_W8_ASYM: return launch_gemv_q_fmt<LEMOQ_QFMT_W8_ASYM>(s32, kch, grid, st, a);
    case LEMOQ_QFMT_W4: return launch_gemv_q_fmt<LEMOQ_QFMT_W4>(s32, kch, grid, st, a);
    case LEMOQ_QFMT_W4_ASYM: return launch_gemv_q_fmt<LEMOQ_QFMT_W4_ASYM>(s32, kch, grid, st, a);
    default: return launch_gemv_q_fmt<LEMOQ_QFMT_MXFP4>(false, kch, grid, st, a);
  }
}

}  // namespace

extern "C" int lemoq_gemv_q_x32(const float* x, int64_t M, int64_t K, const void* qweight, int fmt,
                                const void* scale, const void* zero, int scale_is_f32, int64_t N,
                                int64_t padded_k, int64_t group, void* y, int y_is_f16, void* stream) {
  if (!x || !y) return LEMOQ_ERR_NULL;
  const int rc = check_format(fmt, qweight, scale, zero, scale_is_f32, N, padded_k, group);
  if (rc) return rc;
  if (M <= 0 || M > 65535 || K <= 0 || K > padded_k) return LEMOQ_ERR_SHAPE;
  GemvQ32Args a;
  a.x = x;
  a.x_ld = K;
  a.K = (int)K;
  a.codes = reinterpret_cast<const uint8_t*>(qweight);
  a.row_bytes = (int)(qf_4bit(fmt) ? padded_k / 2 : padded_k);
  a.scale = scale;
  a.zero = zero;
  a.N = N;
  a.ngroups = (int)(padded_k / group);
  a.group = (int)group;
  a.y = y;
  a.y_ld = N;
  a.y_f16 = y_is_f16 ? 1 : 0;
  const int64_t chunks = (a.row_bytes + 1023) / 1024;
  const int kch = chunks <= 1 ? 1 : (chunks <= 2 ? 2 : (chunks <= 4 ? 4 : 8));
  const int64_t blocks = (N + 4 * kGemvQRows - 1) / (4 * kGemvQRows);
  const dim3 grid((unsigned)blocks, (unsigned)M);
  hipStream_t st = lemoq_stream(stream);
  const bool s32 = scale_is_f32 != 0;
  switch (fmt) {
    case LEMOQ_QFMT_W8: return launch_gemv_q_x32_fmt<LEMOQ_QFMT_W8>(s32, kch, grid, st, a);
    case LEMOQ_QFMT_W8_ASYM: return launch_gemv_q_x32_fmt<LEMOQ_QFMT_W8_ASYM>(s32, kch, grid, st, a);
    case LEMOQ_QFMT_W4: return launch_gemv_q_x32_fmt<LEMOQ_QFMT_W4>(s32, kch, grid, st, a);
    case LEMOQ_QFMT_W4_ASYM: return launch_gemv_q_x32_fmt<LEMOQ_QFMT_W4_ASYM>(s32, kch, grid, st, a);
    default: return launch_gemv_q_x32_fmt<LEMOQ_QFMT_MXFP4>(false, kch, grid, st, a);
  }
}

extern "C" int lemoq_dequant_q(const void* qweight, int fmt, const void* scale, const void* zero,
                               int scale_is_f32, int64_t N, int64_t padded_k, int64_t group, void* w,
                               int64_t ld_w, int64_t k_out, int w_is_f32, void* stream) {
  if (!w) return LEMOQ_ERR_NULL;
  const int rc = check_format(fmt, qweight, scale, zero, scale_is_f32, N, padded_k, group);
  if (rc) return rc;
  if (k_out <= 0 || k_out > padded_k || ld_w < k_out) return LEMOQ_ERR_SHAPE;
  DequantQArgs a;
  a.codes = reinterpret_cast<const uint8_t*>(qweight);
  a.row_bytes = (int)(qf_4bit(fmt) ? padded_k / 2 : padded_k);
  a.scale = scale;
  a.zero = zero;
  a.N = N;
  a.ngroups = (int)(padded_k / group);
  a.group = (int)group;
  a.w = w;
  a.ld = ld_w;
  a.k_out = (int)k_out;
  const int64_t slices = N * (a.row_bytes / 16);
  const int64_t blocks = (slices + 255) / 256;
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  const dim3 grid((unsigned)blocks);
  hipStream_t st = lemoq_stream(stream);
  const bool s32 = scale_is_f32 != 0, o32 = w_is_f32 != 0;
  switch (fmt) {
    case LEMOQ_QFMT_W8: return launch_dequant_q<LEMOQ_QFMT_W8>(s32, o32, grid, st, a);
    case LEMOQ_QFMT_W8_ASYM: return launch_dequant_q<LEMOQ_QFMT_W8_ASYM>(s32, o32, grid, st, a);
    case LEMOQ_QFMT_W4: return launch_dequant_q<LEMOQ_QFMT_W4>(s32, o32, grid, st, a);
    case LEMOQ_QFMT_W4_ASYM: return launch_dequant_q<LEMOQ_QFMT_W4_ASYM>(s32, o32, grid, st, a);
    default: return launch_dequant_q<LEMOQ_QFMT_MXFP4>(false, o32, grid, st, a);
  }
}

extern "C" int lemoq_rtn_quantize(const float* w, int64_t rows, int64_t cols, int64_t group, int bits,
                                  int symmetric, uint8_t* codes, uint16_t* scale_f16, float* scale_f32,
                                  uint16_t* zero_f16, float* zero_f32, void* stream) {
  if (!w || !codes) return LEMOQ_ERR_NULL;
  if (bits != 4 && bits != 8) return LEMOQ_ERR_UNSUPPORTED;
  if (rows < 0 || cols <= 0 || group <= 0 || (bits == 4 && group % 2 != 0)) return LEMOQ_ERR_SHAPE;
  if (rows == 0) return LEMOQ_OK;
  const int64_t ngroups = (cols + group - 1) / group;
  const int64_t padded = ngroups * group;
  const int64_t code_ld = bits == 4 ? padded / 2 : padded;
  const int64_t blocks = (rows * ngroups + 3) / 4;
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  hipStream_t st = lemoq_stream(stream);
  const dim3 grid((unsigned)blocks);
#define LEMOQ_RTN_CASE(B, S)                                                                         \
  hipLaunchKernelGGL((rtn_q_kernel<B, S>), grid, dim3(256), 0, st, w, rows, cols, group, ngroups, codes, \
                     code_ld, scale_f16, scale_f32, zero_f16, zero_f32)
  if (bits == 8 && symmetric) LEMOQ_RTN_CASE(8, true);
  else if (bits == 8) LEMOQ_RTN_CASE(8, false);
  else if (symmetric) LEMOQ_RTN_CASE(4, true);
  else LEMOQ_RTN_CASE(4, false);
#undef LEMOQ_RTN_CASE
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_mxfp4_quantize(const float* w, int64_t rows, int64_t cols, uint8_t* codes_packed,
                                    uint8_t* scale_e8m0, void* stream) {
  if (!w || !codes_packed || !scale_e8m0) return LEMOQ_ERR_NULL;
  if (rows < 0 || cols <= 0) return LEMOQ_ERR_SHAPE;
  if (rows == 0) return LEMOQ_OK;
  const int64_t nblk = (cols + 31) / 32;
  const int64_t waves = (rows * nblk + 1) / 2;
  const int64_t blocks = (waves + 3) / 4;
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(mxfp4_quant_kernel, dim3((unsigned)blocks), dim3(256), 0, lemoq_stream(stream), w, rows,
                     cols, nblk, codes_packed, scale_e8m0);
  LEMOQ_CHECK_LAUNCH();
}
