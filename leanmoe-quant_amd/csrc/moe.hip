// Grouped MoE w8a16 GEMVs for one token: top_k of E experts, int8 codes with
// per-group fp16 scales dequantised in registers, fp32 accumulation.
//
// gate/up:  grid (ceil(F / (4*R)), top_k); wave w of block b computes the R
//           gate rows and the R matching up rows n = (4b + w)*R + r of expert
//           ids[slot] and writes act[slot, n] = fp16(silu(g) * u).
// down:     grid ceil(H / R) blocks of 8 waves; wave w walks the slots
//           w, w+8, ... and computes the R rows of expert ids[slot] for the
//           act[slot] vector; the block then sums slot partials * top_w in a
//           fixed slot order (deterministic, no atomics) and applies the
//           optional fp16 residual add.
// Both use the 1 KB-per-row-chunk lane layout of the dense GEMV (gemv.hip).
#include "common.h"

namespace {

template <int KCH>
__device__ __forceinline__ void stage_vec(const uint16_t* __restrict__ src, int n,
                                          uint16_t* __restrict__ xs) {
  constexpr int KP = KCH * 1024;
  for (int i = threadIdx.x * 8; i < KP; i += blockDim.x * 8) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (i < n) v = *reinterpret_cast<const u32x4*>(src + i);
    *reinterpret_cast<u32x4*>(xs + i) = v;
  }
  __syncthreads();
}

template <int KCH, int R>
__global__ __launch_bounds__(256) void moe_gate_up_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ codes,
    const uint16_t* __restrict__ scale, const int64_t* __restrict__ ids, int E, int F, int H,
    int group, uint16_t* __restrict__ act) {
  __shared__ __align__(16) uint16_t xs[KCH * 1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int slot = blockIdx.y;
  stage_vec<KCH>(x, H, xs);
  XChunk xc[KCH];
#pragma unroll
  for (int j = 0; j < KCH; ++j) load_xchunk(xs + 1024 * j + 16 * lane, xc[j]);

  const int64_t e = ids[slot];
  const bool ev = e >= 0 && e < E;
  const int ng = H / group;
  int gidx[KCH];
#pragma unroll
  for (int j = 0; j < KCH; ++j) gidx[j] = (1024 * j + 16 * lane) / group;

  const int n0 = (blockIdx.x * 4 + wave) * R;
  const int64_t ebase = (ev ? e : 0) * (int64_t)(2 * F);
  u32x4 cg[R][KCH], cu[R][KCH];
  float sg[R][KCH], su[R][KCH];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = n0 + r;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int off = 1024 * j + 16 * lane;
      if (ev && n < F && off < H) {
        const int64_t rg = ebase + n, ru = ebase + F + n;
        cg[r][j] = load_stream16(codes + rg * H + off);
        cu[r][j] = load_stream16(codes + ru * H + off);
        sg[r][j] = h2f(scale[rg * ng + gidx[j]]);
        su[r][j] = h2f(scale[ru * ng + gidx[j]]);
      } else {
        cg[r][j] = (u32x4){0u, 0u, 0u, 0u};
        cu[r][j] = (u32x4){0u, 0u, 0u, 0u};
        sg[r][j] = 0.0f;
        su[r][j] = 0.0f;
      }
    }
  }
  float g[R], u[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float ag = 0.0f, au = 0.0f;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      ag = fmaf(sg[r][j], dot16_i8(cg[r][j], xc[j], 0.0f), ag);
      au = fmaf(su[r][j], dot16_i8(cu[r][j], xc[j], 0.0f), au);
    }
    g[r] = wave_sum(ag);
    u[r] = wave_sum(au);
  }
  if (lane < R) {
    float gv = g[0], uv = u[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) {
        gv = g[r];
        uv = u[r];
      }
    const int n = n0 + lane;
    if (n < F) {
      const float sig = 1.0f / (1.0f + expf(-gv));
      act[(int64_t)slot * F + n] = f2h(gv * sig * uv);
    }
  }
}

template <int KCH, int R>
__global__ __launch_bounds__(512) void moe_down_kernel(
    const uint16_t* __restrict__ act, const int8_t* __restrict__ codes,
    const uint16_t* __restrict__ scale, const int64_t* __restrict__ ids,
    const uint16_t* __restrict__ top_w, int top_k, int E, int H, int F, int group,
    const uint16_t* __restrict__ resid, uint16_t* __restrict__ out) {
  __shared__ float part[64][R];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * R;
  const int ng = F / group;
  int gidx[KCH];
#pragma unroll
  for (int j = 0; j < KCH; ++j) gidx[j] = (1024 * j + 16 * lane) / group;

  for (int slot = wave; slot < top_k; slot += 8) {
    const int64_t e = ids[slot];
    const bool ev = e >= 0 && e < E;
    XChunk xc[KCH];
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int off = 1024 * j + 16 * lane;
      if (off < F) {
        load_xchunk(act + (int64_t)slot * F + off, xc[j]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xc[j].a[i] = (f16x2){(f16)0.0f, (f16)0.0f};
          xc[j].b[i] = (f16x2){(f16)0.0f, (f16)0.0f};
        }
      }
    }
    const int64_t ebase = (ev ? e : 0) * (int64_t)H;
    u32x4 c[R][KCH];
    float s[R][KCH];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = n0 + r;
#pragma unroll
      for (int j = 0; j < KCH; ++j) {
        const int off = 1024 * j + 16 * lane;
        if (ev && n < H && off < F) {
          const int64_t row = ebase + n;
          c[r][j] = load_stream16(codes + row * F + off);
          s[r][j] = h2f(scale[row * ng + gidx[j]]);
        } else {
          c[r][j] = (u32x4){0u, 0u, 0u, 0u};
          s[r][j] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < KCH; ++j) a = fmaf(s[r][j], dot16_i8(c[r][j], xc[j], 0.0f), a);
      a = wave_sum(a);
      if (lane == 0) part[slot][r] = a;
    }
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < R) {
    const int n = n0 + t;
    if (n < H) {
      float v = 0.0f;
      for (int i = 0; i < top_k; ++i) v += part[i][t] * h2f(top_w[i]);
      uint16_t o = f2h(v);
      if (resid) o = hadd_round(h2f(o), resid[n]);
      out[n] = o;
    }
  }
}

template <int KCH>
int launch_gate_up(hipStream_t st, const uint16_t* x, const int8_t* codes, const uint16_t* scale,
                   const int64_t* ids, int top_k, int E, int F, int H, int group, uint16_t* act) {
  constexpr int R = 2;
  dim3 grid((unsigned)((F + 4 * R - 1) / (4 * R)), (unsigned)top_k);
  hipLaunchKernelGGL((moe_gate_up_kernel<KCH, R>), grid, dim3(256), 0, st, x, codes, scale, ids, E,
                     F, H, group, act);
  LEMOQ_CHECK_LAUNCH();
}

template <int KCH>
int launch_down(hipStream_t st, const uint16_t* act, const int8_t* codes, const uint16_t* scale,
                const int64_t* ids, const uint16_t* top_w, int top_k, int E, int H, int F,
                int group, const uint16_t* resid, uint16_t* out) {
  constexpr int R = 4;
  dim3 grid((unsigned)((H + R - 1) / R));
  hipLaunchKernelGGL((moe_down_kernel<KCH, R>), grid, dim3(512), 0, st, act, codes, scale, ids,
                     top_w, top_k, E, H, F, group, resid, out);
  LEMOQ_CHECK_LAUNCH();
}

int kch_of(int64_t k) {
  const int64_t c = (k + 1023) / 1024;
  return c <= 1 ? 1 : (c <= 2 ? 2 : (c <= 4 ? 4 : 8));
}

}  // namespace

extern "C" int lemoq_moe_gate_up_w8(const uint16_t* x, const int8_t* codes, const uint16_t* scale,
                                    const int64_t* ids, int64_t top_k, int64_t num_experts,
                                    int64_t ffn, int64_t hidden, int64_t group, uint16_t* act,
                                    void* stream) {
  if (!x || !codes || !scale || !ids || !act) return LEMOQ_ERR_NULL;
  if (top_k <= 0 || top_k > 65535 || num_experts <= 0 || ffn <= 0 || hidden <= 0)
    return LEMOQ_ERR_SHAPE;
  if (hidden > 8192 || hidden % 16 != 0 || group <= 0 || group % 16 != 0 || hidden % group != 0)
    return LEMOQ_ERR_UNSUPPORTED;
  if (num_experts * 2 * ffn * hidden >= (int64_t)1 << 40) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(codes) || !lemoq_aligned16(x)) return LEMOQ_ERR_ALIGN;
  hipStream_t st = lemoq_stream(stream);
  switch (kch_of(hidden)) {
    case 1: return launch_gate_up<1>(st, x, codes, scale, ids, (int)top_k, (int)num_experts, (int)ffn, (int)hidden, (int)group, act);
    case 2: return launch_gate_up<2>(st, x, codes, scale, ids, (int)top_k, (int)num_experts, (int)ffn, (int)hidden, (int)group, act);
    case 4: return launch_gate_up<4>(st, x, codes, scale, ids, (int)top_k, (int)num_experts, (int)ffn, (int)hidden, (int)group, act);
    default: return launch_gate_up<8>(st, x, codes, scale, ids, (int)top_k, (int)num_experts, (int)ffn, (int)hidden, (int)group, act);
  }
}

extern "C" int lemoq_moe_down_w8(const uint16_t* act, const int8_t* codes, const uint16_t* scale,
                                 const int64_t* ids, const uint16_t* top_w, int64_t top_k,
                                 int64_t num_experts, int64_t hidden, int64_t ffn, int64_t group,
                                 const uint16_t* residual, uint16_t* out, void* stream) {
  if (!act || !codes || !scale || !ids || !top_w || !out) return LEMOQ_ERR_NULL;
  if (top_k <= 0 || top_k > 64 || num_experts <= 0 || ffn <= 0 || hidden <= 0)
    return LEMOQ_ERR_SHAPE;
  if (ffn > 8192 || ffn % 16 != 0 || group <= 0 || group % 16 != 0 || ffn % group != 0)
    return LEMOQ_ERR_UNSUPPORTED;
  if (num_experts * hidden * ffn >= (int64_t)1 << 40) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(codes) || !lemoq_aligned16(act)) return LEMOQ_ERR_ALIGN;
  hipStream_t st = lemoq_stream(stream);
  switch (kch_of(ffn)) {
    case 1: return launch_down<1>(st, act, codes, scale, ids, top_w, (int)top_k, (int)num_experts, (int)hidden, (int)ffn, (int)group, residual, out);
    case 2: return launch_down<2>(st, act, codes, scale, ids, top_w, (int)top_k, (int)num_experts, (int)hidden, (int)ffn, (int)group, residual, out);
    case 4: return launch_down<4>(st, act, codes, scale, ids, top_w, (int)top_k, (int)num_experts, (int)hidden, (int)ffn, (int)group, residual, out);
    default: return launch_down<8>(st, act, codes, scale, ids, top_w, (int)top_k, (int)num_experts, (int)hidden, (int)ffn, (int)group, residual, out);
  }
}
