// w8a16 dense GEMV (dequantisation in registers), the fused router
// (RMSNorm + fp16 GEMV + softmax/top-k), routing top-k and the greedy argmax
// that advances the decode position on the device.
//
// GEMV layout.  A 256-thread block is 4 waves; each wave owns R consecutive
// output rows.  A row of K int8 codes is read as K/1024 chunks of 1 KB: lane l
// loads the 16 bytes at 1024*j + 16*l (one global_load_dwordx4, fully
// coalesced), so a lane's 16 codes always sit inside one quantisation group
// (group % 16 == 0) and it needs exactly one fp16 scale per chunk.  The
// activation row is staged once per block in LDS (with the RMSNorm prologue
// applied there when requested) and each lane keeps its own 16*K/1024 values
// in registers, pre-permuted for v_dot2_f32_f16.  After the loads of all R
// rows are issued, each lane forms s * sum(c*x) per chunk and a wave
// butterfly reduces the row.  No MFMA: at batch 1 this is ~1 flop/byte and
// HBM bound.
#include "common.h"

namespace {

// Stage x[0:K) (fp16) into LDS xs[0:KCH*1024), zero padded; optionally apply
// the HF RMSNorm (fp32 mean of squares, x*rstd rounded to fp16, times the
// fp16 weight with one rounding).  Returns after a block barrier.
template <int KCH>
__device__ __forceinline__ void stage_x(const uint16_t* __restrict__ xr, int K,
                                        const uint16_t* __restrict__ norm_w, float eps,
                                        uint16_t* __restrict__ x_copy, bool write_copy,
                                        uint16_t* __restrict__ xs, float* __restrict__ red) {
  const int tid = threadIdx.x;
  constexpr int KP = KCH * 1024;
  const bool vec = ((K & 7) == 0) && ((reinterpret_cast<uintptr_t>(xr) & 15u) == 0);
  float ssq = 0.0f;
  if (vec) {
    for (int i = tid * 8; i < KP; i += 256 * 8) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (i < K) v = *reinterpret_cast<const u32x4*>(xr + i);
      *reinterpret_cast<u32x4*>(xs + i) = v;
      if (norm_w) {
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float a = h2f((uint16_t)(w4[q] & 0xFFFFu));
          const float b = h2f((uint16_t)(w4[q] >> 16));
          ssq += a * a;
          ssq += b * b;
        }
      }
      if (write_copy && i < K) *reinterpret_cast<u32x4*>(x_copy + i) = v;
    }
  } else {
    for (int i = tid; i < KP; i += 256) {
      const uint16_t v = i < K ? xr[i] : (uint16_t)0;
      xs[i] = v;
      if (norm_w) {
        const float a = h2f(v);
        ssq += a * a;
      }
      if (write_copy && i < K) x_copy[i] = v;
    }
  }
  if (norm_w) {
    ssq = wave_sum(ssq);
    if ((tid & 63) == 0) red[tid >> 6] = ssq;
    __syncthreads();
    const float tot = red[0] + red[1] + red[2] + red[3];
    const float rstd = 1.0f / sqrtf(tot / (float)K + eps);
    for (int i = tid; i < K; i += 256) {
      const uint16_t nh = f2h(h2f(xs[i]) * rstd);
      xs[i] = f2h(h2f(nh) * h2f(norm_w[i]));
    }
  }
  __syncthreads();
}

template <int KCH, int R>
__global__ __launch_bounds__(256) void gemv_w8_kernel(
    const uint16_t* __restrict__ x, int64_t x_ld, const int64_t* __restrict__ x_row_index,
    int64_t x_rows, int K, const uint16_t* __restrict__ norm_w, float eps,
    uint16_t* __restrict__ x_copy, const int8_t* __restrict__ codes,
    const uint16_t* __restrict__ scale, int64_t N, int Kp, int group,
    const uint16_t* __restrict__ resid, void* __restrict__ y, int64_t y_ld, int y_f16) {
  __shared__ __align__(16) uint16_t xs[KCH * 1024];
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t m = blockIdx.y;

  const uint16_t* xr;
  bool x_valid = true;
  if (x_row_index) {
    const int64_t r = x_row_index[0];
    x_valid = r >= 0 && r < x_rows;
    xr = x + (x_valid ? r : 0) * x_ld;
  } else {
    xr = x + m * x_ld;
  }
  stage_x<KCH>(xr, x_valid ? K : 0, norm_w, eps, x_copy, x_copy != nullptr && blockIdx.x == 0,
               xs, red);

  XChunk xc[KCH];
#pragma unroll
  for (int j = 0; j < KCH; ++j) load_xchunk(xs + 1024 * j + 16 * lane, xc[j]);

  const int ngroups = Kp / group;
  int gidx[KCH];
#pragma unroll
  for (int j = 0; j < KCH; ++j) gidx[j] = (1024 * j + 16 * lane) / group;

  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * R;
  u32x4 c[R][KCH];
  float s[R][KCH];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t n = row0 + r;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int off = 1024 * j + 16 * lane;
      if (n < N && off < Kp) {
        c[r][j] = load_stream16(codes + n * Kp + off);
        s[r][j] = h2f(scale[n * ngroups + gidx[j]]);
      } else {
        c[r][j] = (u32x4){0u, 0u, 0u, 0u};
        s[r][j] = 0.0f;
      }
    }
  }
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < KCH; ++j) a = fmaf(s[r][j], dot16_i8(c[r][j], xc[j], 0.0f), a);
    acc[r] = wave_sum(a);
  }
  if (lane < R) {
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) v = acc[r];
    const int64_t n = row0 + lane;
    if (n < N) {
      if (y_f16) {
        uint16_t o = f2h(v);
        if (resid) o = hadd_round(h2f(o), resid[n]);
        reinterpret_cast<uint16_t*>(y)[m * y_ld + n] = o;
      } else {
        reinterpret_cast<float*>(y)[m * y_ld + n] = v;
      }
    }
  }
}

template <int KCH>
int launch_gemv(int R, dim3 grid, hipStream_t st, const uint16_t* x, int64_t x_ld,
                const int64_t* x_row_index, int64_t x_rows, int K, const uint16_t* norm_w,
                float eps, uint16_t* x_copy, const int8_t* codes, const uint16_t* scale,
                int64_t N, int Kp, int group, const uint16_t* resid, void* y, int64_t y_ld,
                int y_f16) {
#define LEMOQ_GEMV_CASE(RR)                                                                      \
  case RR:                                                                                       \
    hipLaunchKernelGGL((gemv_w8_kernel<KCH, RR>), grid, dim3(256), 0, st, x, x_ld, x_row_index, \
                       x_rows, K, norm_w, eps, x_copy, codes, scale, N, Kp, group, resid, y,    \
                       y_ld, y_f16);                                                             \
    break;
  switch (R) {
    LEMOQ_GEMV_CASE(1)
    LEMOQ_GEMV_CASE(2)
    LEMOQ_GEMV_CASE(4)
    default: return LEMOQ_ERR_UNSUPPORTED;
  }
#undef LEMOQ_GEMV_CASE
  LEMOQ_CHECK_LAUNCH();
}

int rows_per_wave(int64_t N) { return N <= 4096 ? 1 : (N <= 16384 ? 2 : 4); }

int gemv_dispatch(hipStream_t st, const uint16_t* x, int64_t x_ld, const int64_t* x_row_index,
                  int64_t x_rows, int64_t M, int64_t K, const uint16_t* norm_w, float eps,
                  uint16_t* x_copy, const int8_t* codes, const uint16_t* scale, int64_t N,
                  int64_t Kp, int64_t group, const uint16_t* resid, void* y, int64_t y_ld,
                  int y_f16) {
  if (N <= 0 || M <= 0 || K <= 0) return LEMOQ_ERR_SHAPE;
  if (Kp > 8192 || Kp % 16 != 0 || group <= 0 || group % 16 != 0 || Kp % group != 0 || K > Kp)
    return LEMOQ_ERR_UNSUPPORTED;
  if (M > 65535) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(codes)) return LEMOQ_ERR_ALIGN;
  const int R = rows_per_wave(N);
  const int64_t blocks = (N + 4 * R - 1) / (4 * R);
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  dim3 grid((unsigned)blocks, (unsigned)M);
  const int kch = (int)((Kp + 1023) / 1024);
  const int kch_pow2 = kch <= 1 ? 1 : (kch <= 2 ? 2 : (kch <= 4 ? 4 : 8));
  switch (kch_pow2) {
    case 1:
      return launch_gemv<1>(R, grid, st, x, x_ld, x_row_index, x_rows, (int)K, norm_w, eps,
                            x_copy, codes, scale, N, (int)Kp, (int)group, resid, y, y_ld, y_f16);
    case 2:
      return launch_gemv<2>(R, grid, st, x, x_ld, x_row_index, x_rows, (int)K, norm_w, eps,
                            x_copy, codes, scale, N, (int)Kp, (int)group, resid, y, y_ld, y_f16);
    case 4:
      return launch_gemv<4>(R, grid, st, x, x_ld, x_row_index, x_rows, (int)K, norm_w, eps,
                            x_copy, codes, scale, N, (int)Kp, (int)group, resid, y, y_ld, y_f16);
    default:
      return launch_gemv<8>(R, grid, st, x, x_ld, x_row_index, x_rows, (int)K, norm_w, eps,
                            x_copy, codes, scale, N, (int)Kp, (int)group, resid, y, y_ld, y_f16);
  }
}

}  // namespace

extern "C" int lemoq_gemv_w8(const uint16_t* x, int64_t M, int64_t K, const int8_t* codes,
                             const uint16_t* scale, int64_t N, int64_t padded_k, int64_t group,
                             void* y, int y_is_f16, void* stream) {
  if (!x || !codes || !scale || !y) return LEMOQ_ERR_NULL;
  return gemv_dispatch(lemoq_stream(stream), x, K, nullptr, 0, M, K, nullptr, 0.0f, nullptr,
                       codes, scale, N, padded_k, group, nullptr, y, N, y_is_f16 ? 1 : 0);
}

extern "C" int lemoq_gemv_w8_fused(const uint16_t* x_src, const int64_t* x_row_index,
                                   int64_t x_rows, const uint16_t* norm_w, float eps,
                                   uint16_t* x_copy, const int8_t* codes, const uint16_t* scale,
                                   int64_t N, int64_t K, int64_t group, const uint16_t* residual,
                                   uint16_t* y, void* stream) {
  if (!x_src || !codes || !scale || !y) return LEMOQ_ERR_NULL;
  if (x_row_index && x_rows <= 0) return LEMOQ_ERR_SHAPE;
  return gemv_dispatch(lemoq_stream(stream), x_src, K, x_row_index, x_rows, 1, K, norm_w, eps,
                       x_copy, codes, scale, N, K, group, residual, y, N, 1);
}

// ---------------------------------------------------------------------------
// Routing: softmax over E values then top_k by probability (ties -> lowest
// index), optional renormalisation.  One wave handles one token; lane l holds
// values l, l+64, ... (E <= 1024).  Arithmetic follows
// src/lemoq/kernels/_routing_triton.py:55-80 and moe_static._route
// (src/lemoq/kernels/moe_static.py:276-283): p = exp(z - max) / sum(exp(z - max)).
// ---------------------------------------------------------------------------
namespace {
constexpr int kMaxPerLane = 16;  // E <= 1024

__device__ void wave_route_topk(const float (&z)[kMaxPerLane], int E, int top_k, bool norm,
                                float* __restrict__ out_w32, uint16_t* __restrict__ out_w16,
                                int64_t* __restrict__ out_i) {
  const int lane = threadIdx.x & 63;
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i)
    if (lane + 64 * i < E) mx = fmaxf(mx, z[i]);
  mx = wave_max(mx);
  float p[kMaxPerLane];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    p[i] = (lane + 64 * i < E) ? expf(z[i] - mx) : 0.0f;
    sum += p[i];
  }
  sum = wave_sum(sum);
  uint32_t taken = 0u;  // bit i: element lane+64*i already selected
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) p[i] = (lane + 64 * i < E) ? p[i] / sum : -1.0f;
  float wsel = 0.0f;  // lane k < top_k keeps the k-th selected probability
  float wsum = 0.0f;
  for (int k = 0; k < top_k; ++k) {
    float bv = -2.0f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
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
    if (lane == k) wsel = bv;
    wsum += bv;
    if (lane == 0) out_i[k] = (int64_t)bi;
  }
  if (lane < top_k) {
    const float w = norm ? wsel / wsum : wsel;
    if (out_w32) out_w32[lane] = w;
    if (out_w16) out_w16[lane] = f2h(w);
  }
}

__global__ __launch_bounds__(256) void route_topk_kernel(const void* __restrict__ logits, int f16,
                                                         int64_t T, int E, int64_t stride,
                                                         int top_k, int norm,
                                                         float* __restrict__ top_w,
                                                         int64_t* __restrict__ top_i) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int lane = threadIdx.x & 63;
  float z[kMaxPerLane];
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int idx = lane + 64 * i;
    if (idx < E) {
      z[i] = f16 ? h2f(reinterpret_cast<const uint16_t*>(logits)[t * stride + idx])
                 : reinterpret_cast<const float*>(logits)[t * stride + idx];
    } else {
      z[i] = -INFINITY;
    }
  }
  wave_route_topk(z, E, top_k, norm != 0, top_w + t * top_k, nullptr, top_i + t * top_k);
}

// Fused router of one token: 16 waves.  RMSNorm of h into LDS (and xn_out),
// fp16 GEMV over E rows (lane l reads 8 fp16 at 8*l + 512*i: 16-byte loads),
// logits rounded once to fp16, then wave 0 routes.
__global__ __launch_bounds__(1024) void router_fused_kernel(
    const uint16_t* __restrict__ h, const uint16_t* __restrict__ norm_w, float eps, int H,
    const uint16_t* __restrict__ rw, int E, int top_k, int norm, uint16_t* __restrict__ xn_out,
    uint16_t* __restrict__ logits_out, float* __restrict__ top_w32,
    uint16_t* __restrict__ top_w16, int64_t* __restrict__ top_i) {
  __shared__ __align__(16) uint16_t xs[8192];
  __shared__ float red[16];
  __shared__ float lg[1024];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float ssq = 0.0f;
  for (int i = tid; i < H; i += 1024) {
    const uint16_t v = h[i];
    xs[i] = v;
    const float a = h2f(v);
    ssq += a * a;
  }
  if (norm_w) {
    ssq = wave_sum(ssq);
    if (lane == 0) red[wave] = ssq;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < 16; ++w) tot += red[w];
    const float rstd = 1.0f / sqrtf(tot / (float)H + eps);
    for (int i = tid; i < H; i += 1024) {
      const uint16_t nh = f2h(h2f(xs[i]) * rstd);
      xs[i] = f2h(h2f(nh) * h2f(norm_w[i]));
    }
  }
  __syncthreads();
  if (xn_out)
    for (int i = tid; i < H; i += 1024) xn_out[i] = xs[i];
  for (int e = wave; e < E; e += 16) {
    const uint16_t* wr = rw + (int64_t)e * H;
    float a = 0.0f;
    for (int k = 8 * lane; k < H; k += 512) {
      const u32x4 wv = *reinterpret_cast<const u32x4*>(wr + k);
      const u32x4 xv = *reinterpret_cast<const u32x4*>(xs + k);
      const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) a = __builtin_amdgcn_fdot2(as_h2(ww[i]), as_h2(xw[i]), a, false);
    }
    a = wave_sum(a);
    if (lane == 0) {
      const uint16_t lh = f2h(a);
      lg[e] = h2f(lh);
      if (logits_out) logits_out[e] = lh;
    }
  }
  __syncthreads();
  if (wave == 0) {
    float z[kMaxPerLane];
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) z[i] = (lane + 64 * i < E) ? lg[lane + 64 * i] : -INFINITY;
    wave_route_topk(z, E, top_k, norm != 0, top_w32, top_w16, top_i);
  }
}

// Greedy argmax (first index on ties) + step advance, one 1024-thread block.
__global__ __launch_bounds__(1024) void argmax_advance_kernel(
    const uint16_t* __restrict__ logits, int64_t n, int64_t* __restrict__ token,
    int64_t* __restrict__ pos, int32_t* __restrict__ filled, const int64_t* __restrict__ prompt,
    int64_t prompt_len, int64_t* __restrict__ history, int64_t history_len) {
  __shared__ float bvs[16];
  __shared__ int64_t bis[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float bv = -INFINITY;
  int64_t bi = n;  // sentinel larger than every index
  for (int64_t i = tid; i < n; i += 1024) {
    const float v = h2f(logits[i]);
    if (v > bv) {  // ascending scan: strict > keeps the first index
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int64_t oi = __shfl_xor(bi, o, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    bvs[wave] = bv;
    bis[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = bvs[0];
    int64_t idx = bis[0];
    for (int w = 1; w < 16; ++w) {
      if (bvs[w] > v || (bvs[w] == v && bis[w] < idx)) {
        v = bvs[w];
        idx = bis[w];
      }
    }
    if (idx >= n) idx = 0;  // every logit was -inf or NaN
    const int64_t p = pos[0];
    int64_t next = idx;
    if (prompt && p + 1 < prompt_len) next = prompt[p + 1];
    token[0] = next;
    if (history && p + 1 >= 0 && p + 1 < history_len) history[p + 1] = next;
    pos[0] = p + 1;
    filled[0] = (int32_t)(p + 2);
  }
}

}  // namespace

extern "C" int lemoq_route_topk(const void* logits, int logits_is_f16, int64_t T, int64_t E,
                                int64_t row_stride, int64_t top_k, int norm_topk_prob,
                                float* top_w, int64_t* top_i, void* stream) {
  if (!logits || !top_w || !top_i) return LEMOQ_ERR_NULL;
  if (T < 0 || E <= 0 || E > 1024 || top_k <= 0 || top_k > E || top_k > 64 || row_stride < E)
    return LEMOQ_ERR_SHAPE;
  if (T == 0) return LEMOQ_OK;
  const int64_t blocks = (T + 3) / 4;
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(route_topk_kernel, dim3((unsigned)blocks), dim3(256), 0, lemoq_stream(stream),
                     logits, logits_is_f16 ? 1 : 0, T, (int)E, row_stride, (int)top_k,
                     norm_topk_prob ? 1 : 0, top_w, top_i);
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_router_topk_fused(const uint16_t* h, const uint16_t* norm_w, float eps,
                                       int64_t hidden, const uint16_t* router_w, int64_t E,
                                       int64_t top_k, int norm_topk_prob, uint16_t* xn_out,
                                       uint16_t* logits_out, float* top_w_f32,
                                       uint16_t* top_w_f16, int64_t* top_i, void* stream) {
  if (!h || !router_w || !top_i) return LEMOQ_ERR_NULL;
  if (hidden <= 0 || hidden > 8192 || hidden % 8 != 0) return LEMOQ_ERR_UNSUPPORTED;
  if (E <= 0 || E > 1024 || top_k <= 0 || top_k > E || top_k > 64) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(router_w)) return LEMOQ_ERR_ALIGN;
  hipLaunchKernelGGL(router_fused_kernel, dim3(1), dim3(1024), 0, lemoq_stream(stream), h, norm_w,
                     eps, (int)hidden, router_w, (int)E, (int)top_k, norm_topk_prob ? 1 : 0,
                     xn_out, logits_out, top_w_f32, top_w_f16, top_i);
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_argmax_advance(const uint16_t* logits, int64_t n, int64_t* token,
                                    int64_t* pos, int32_t* filled, const int64_t* prompt,
                                    int64_t prompt_len, int64_t* history, int64_t history_len,
                                    void* stream) {
  if (!logits || !token || !pos || !filled) return LEMOQ_ERR_NULL;
  if (n <= 0) return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(argmax_advance_kernel, dim3(1), dim3(1024), 0, lemoq_stream(stream), logits,
                     n, token, pos, filled, prompt, prompt_len, history, history_len);
  LEMOQ_CHECK_LAUNCH();
}
