// Grouped MoE GEMVs for one token on 4-bit symmetric experts: top_k of E
// experts, int4 codes packed two per byte (the even column in the low nibble)
// with per-group fp16 scales, fp32 accumulation.  The 4-bit branch of the
// reference's grouped kernels (_gate_up_act_kernel_q / _down_sum_kernel_q
// with BITS=4, src/lemoq/kernels/_grouped_triton.py:235-398, nibbles expanded
// by _expand_int4 :235-247) and of quantize_fused_experts(bits=4)
// (src/lemoq/kernels/moe_grouped_quant.py:191-244).
//
// Same structure and numerics as the 8-bit kernels (moe.hip): gate/up grid
// (ceil(F / (4R)), top_k), wave w of block b computes the R gate rows and the
// R matching up rows of expert ids[slot] and writes act = fp16(silu(g) * u);
// down grid ceil(H / R) blocks of 8 waves walking the slots, then a
// fixed-order sum of partial * top_w and the optional fp16 residual add.
// Lane l reads bytes [1024 j + 16 l, +16) of chunk j of a packed row (32
// codes) and the matching 32 activations; codes become exact fp16 values
// (nibble masks, byte permutes against 0x64, one packed subtract) dotted with
// v_dot2_f32_f16.
#include "qformat.h"

namespace {

using namespace lemoq_qf;

// One packed row tile of R rows: KCH 16-byte slices per row and their scales.
template <int R, int KCH>
struct Q4Tile {
  u32x4 c[R][KCH];
  uint16_t s[R][KCH];
  uint32_t ok;
};

template <int R, int KCH>
__device__ __forceinline__ void q4_issue(Q4Tile<R, KCH>& t, const uint8_t* __restrict__ codes,
                                         const uint16_t* __restrict__ scale, int64_t row0, int64_t nrows,
                                         int row_bytes, int ngroups, int group, int lane) {
  t.ok = 0u;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = row0 + r;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int off = 1024 * j + 16 * lane;
      const bool in = row < nrows && off < row_bytes;
      const int64_t rr = in ? row : 0;
      const int oo = in ? off : 0;
      t.c[r][j] = load_stream16(reinterpret_cast<const int8_t*>(codes) + rr * row_bytes + oo);
      t.s[r][j] = scale[rr * ngroups + (oo * 2) / group];
      t.ok |= (in ? 1u : 0u) << (r * KCH + j);
    }
  }
}

template <int KCH>
struct X4 {
  XChunk a[KCH], b[KCH];  // activations [2048 j + 32 l, +16) and [+16, +32)
};

template <int KCH>
__device__ __forceinline__ void x4_load(uint32_t (&w)[KCH][16], const uint16_t* __restrict__ x, int n, int lane) {
  const bool vec = ((reinterpret_cast<uintptr_t>(x) & 15u) == 0) && ((n & 7) == 0);
#pragma unroll
  for (int j = 0; j < KCH; ++j) xq_load<32>(w[j], x, n, 2048 * j + 32 * lane, vec);
}

template <int KCH>
__device__ __forceinline__ void x4_chunks(const uint32_t (&w)[KCH][16], X4<KCH>& x) {
#pragma unroll
  for (int j = 0; j < KCH; ++j) {
    xchunk_of(&w[j][0], x.a[j]);
    xchunk_of(&w[j][8], x.b[j]);
  }
}

template <int R, int KCH>
__device__ __forceinline__ float q4_row_dot(const Q4Tile<R, KCH>& t, int r, const X4<KCH>& x) {
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < KCH; ++j) {
    const float sc = ((t.ok >> (r * KCH + j)) & 1u) ? h2f(t.s[r][j]) : 0.0f;
    a = fmaf(sc, dot32_i4<true>(t.c[r][j], x.a[j], x.b[j], 0.0f), a);
  }
  return a;
}

template <int KCH, int R>
__global__ __launch_bounds__(256) void moe_gate_up_q4_kernel(const uint16_t* __restrict__ x,
                                                             const uint8_t* __restrict__ codes,
                                                             const uint16_t* __restrict__ scale,
                                                             const int64_t* __restrict__ ids, int E, int F, int H,
                                                             int group, uint16_t* __restrict__ act) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int slot = blockIdx.y;
  const int64_t e = ids[slot];
  uint32_t xw[KCH][16];
  x4_load<KCH>(xw, x, H, lane);
  const bool ev = e >= 0 && e < E;
  const int n0 = (blockIdx.x * 4 + wave) * R;
  const int ng = H / group;
  const int rb = H / 2;
  const int64_t ebase = (ev ? e : 0) * (int64_t)(2 * F);
  const int64_t nrows = ev ? (int64_t)F : 0;  // an invalid expert id yields a zero row
  Q4Tile<R, KCH> tg, tu;
  q4_issue<R, KCH>(tg, codes + ebase * rb, scale + ebase * ng, n0, nrows, rb, ng, group, lane);
  q4_issue<R, KCH>(tu, codes + (ebase + F) * rb, scale + (ebase + F) * ng, n0, nrows, rb, ng, group, lane);
  LEMOQ_LOADS_ISSUED();
  X4<KCH> xc;
  x4_chunks<KCH>(xw, xc);
  float g[R], u[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    g[r] = wave_sum(q4_row_dot<R, KCH>(tg, r, xc));
    u[r] = wave_sum(q4_row_dot<R, KCH>(tu, r, xc));
  }
  if (lane < R) {
    float gv = g[0], uv = u[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) {
        gv = g[r];
        uv = u[r];
      }
    if (!ev) gv = uv = 0.0f;
    const int n = n0 + lane;
    if (n < F) {
      const float sig = 1.0f / (1.0f + expf(-gv));
      act[(int64_t)slot * F + n] = f2h(gv * sig * uv);
    }
  }
}

template <int KCH, int R>
__global__ __launch_bounds__(512) void moe_down_q4_kernel(
    const uint16_t* __restrict__ act, const uint8_t* __restrict__ codes, const uint16_t* __restrict__ scale,
    const int64_t* __restrict__ ids, const uint16_t* __restrict__ top_w, int top_k, int E, int H, int F,
    int group, const uint16_t* __restrict__ resid, uint16_t* __restrict__ out) {
  __shared__ float part[64][R];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * R;
  const int ng = F / group;
  const int rb = F / 2;
  const int t = threadIdx.x;
  const int nres = n0 + (t & (R - 1));
  const uint16_t res = *(resid ? resid + (nres < H ? nres : H - 1) : act);
  for (int slot = wave; slot < top_k; slot += 8) {
    const int64_t e = ids[slot];
    const float wslot = h2f(top_w[slot]);
    uint32_t aw[KCH][16];
    x4_load<KCH>(aw, act + (int64_t)slot * F, F, lane);
    const bool ev = e >= 0 && e < E;
    const int64_t ebase = (ev ? e : 0) * (int64_t)H;
    Q4Tile<R, KCH> tl;
    q4_issue<R, KCH>(tl, codes + ebase * rb, scale + ebase * ng, n0, ev ? (int64_t)H : 0, rb, ng, group, lane);
    LEMOQ_LOADS_ISSUED();
    X4<KCH> xc;
    x4_chunks<KCH>(aw, xc);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = wave_sum(q4_row_dot<R, KCH>(tl, r, xc));
      if (lane == 0) part[slot][r] = ev ? v * wslot : 0.0f;
    }
  }
  __syncthreads();
  if (t < R) {
    const int n = n0 + t;
    if (n < H) {
      float v = 0.0f;
      for (int i = 0; i < top_k; ++i) v += part[i][t];
      uint16_t o = f2h(v);
      if (resid) o = hadd_round(h2f(o), res);
      out[n] = o;
    }
  }
}

int kch4_of(int64_t k) {  // 1 KB chunks of a packed 4-bit row of k codes
  const int64_t c = (k / 2 + 1023) / 1024;
  return c <= 1 ? 1 : (c <= 2 ? 2 : 4);
}

}  // namespace

extern "C" int lemoq_moe_gate_up_w4(const uint16_t* x, const uint8_t* codes, const uint16_t* scale,
                                    const int64_t* ids, int64_t top_k, int64_t num_experts, int64_t ffn,
                                    int64_t hidden, int64_t group, uint16_t* act, void* stream) {
  if (!x || !codes || !scale || !ids || !act) return LEMOQ_ERR_NULL;
  if (top_k <= 0 || top_k > 65535 || num_experts <= 0 || ffn <= 0 || hidden <= 0) return LEMOQ_ERR_SHAPE;
  if (hidden > 8192 || hidden % 32 != 0 || group <= 0 || group % 32 != 0 || hidden % group != 0)
    return LEMOQ_ERR_UNSUPPORTED;
  if (num_experts * 2 * ffn * hidden >= (int64_t)1 << 40) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(codes)) return LEMOQ_ERR_ALIGN;
  constexpr int R = 2;
  const dim3 grid((unsigned)((ffn + 4 * R - 1) / (4 * R)), (unsigned)top_k);
  hipStream_t st = lemoq_stream(stream);
  const int E = (int)num_experts, F = (int)ffn, H = (int)hidden, g = (int)group;
  switch (kch4_of(hidden)) {
    case 1: hipLaunchKernelGGL((moe_gate_up_q4_kernel<1, R>), grid, dim3(256), 0, st, x, codes, scale, ids, E, F, H, g, act); break;
    case 2: hipLaunchKernelGGL((moe_gate_up_q4_kernel<2, R>), grid, dim3(256), 0, st, x, codes, scale, ids, E, F, H, g, act); break;
    default: hipLaunchKernelGGL((moe_gate_up_q4_kernel<4, R>), grid, dim3(256), 0, st, x, codes, scale, ids, E, F, H, g, act); break;
  }
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_moe_down_w4(const uint16_t* act, const uint8_t* codes, const uint16_t* scale,
                                 const int64_t* ids, const uint16_t* top_w, int64_t top_k, int64_t num_experts,
                                 int64_t hidden, int64_t ffn, int64_t group, const uint16_t* residual,
                                 uint16_t* out, void* stream) {
  if (!act || !codes || !scale || !ids || !top_w || !out) return LEMOQ_ERR_NULL;
  if (top_k <= 0 || top_k > 64 || num_experts <= 0 || ffn <= 0 || hidden <= 0) return LEMOQ_ERR_SHAPE;
  if (ffn > 8192 || ffn % 32 != 0 || group <= 0 || group % 32 != 0 || ffn % group != 0)
    return LEMOQ_ERR_UNSUPPORTED;
  if (num_experts * hidden * ffn >= (int64_t)1 << 40) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(codes)) return LEMOQ_ERR_ALIGN;
  constexpr int R = 4;
  const dim3 grid((unsigned)((hidden + R - 1) / R));
  hipStream_t st = lemoq_stream(stream);
  const int K = (int)top_k, E = (int)num_experts, H = (int)hidden, F = (int)ffn, g = (int)group;
  switch (kch4_of(ffn)) {
    case 1: hipLaunchKernelGGL((moe_down_q4_kernel<1, R>), grid, dim3(512), 0, st, act, codes, scale, ids, top_w, K, E, H, F, g, residual, out); break;
    case 2: hipLaunchKernelGGL((moe_down_q4_kernel<2, R>), grid, dim3(512), 0, st, act, codes, scale, ids, top_w, K, E, H, F, g, residual, out); break;
    default: hipLaunchKernelGGL((moe_down_q4_kernel<4, R>), grid, dim3(512), 0, st, act, codes, scale, ids, top_w, K, E, H, F, g, residual, out); break;
  }
  LEMOQ_CHECK_LAUNCH();
}
