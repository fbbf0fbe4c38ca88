// Fused per-layer attention of the decode step over the KV-INT8 cache: one
// 1024-thread block (16 waves) per head does
//   q_norm / k_norm (RMSNorm over all heads*D values, HF rounding points),
//   RoPE at *pos, the KV-INT8 write of the new k/v row to slot *pos, and the
//   softmax attention of q over tokens [0, *pos] with the per-token scales
//   folded in (score = ((q.c) * qk_scale) * ks, acc += (p * vs) * c, l += p),
// and writes the head's fp16 output.  One block per head needs no split merge
// (a cross-block reduction would need another launch: on MI355X a kernel
// boundary inside a graph costs ~1.6 us, a grid barrier or "last block"
// atomic more), so it replaces three launches of the split path
// (qk_norm_rope_kv_i8, attn_split_i8, attn_merge) while the cache fits the
// per-CU bandwidth (the step uses it up to 8192 cache slots).
//
// Waves 0-2 compute the q row, the new k row (quantised: written to the cache
// and kept in LDS) and the new v row while waves 3-15 already stream their
// first 64 cached tokens; the first block of cache loads of every wave is
// issued before *pos is known (addresses clamped to the capacity, validity
// decided afterwards), so one memory round trip starts everything.  Cached
// tokens [0, pos) are read from memory; the new token is folded in by wave 0
// from LDS (the same int8 codes and fp16 scale the cache now holds), never
// read back from the cache it just wrote.
//
// Arithmetic restates the reference's patched attention
// (src/lemoq/kernels/attn_decode.py:882-1000), _attn_split_kernel_int8
// (src/lemoq/kernels/_attn_triton.py:102-165), the KV write
// (src/lemoq/kernels/kv_int8.py:196-216) and _rope_one_kernel
// (src/lemoq/kernels/rope.py:101-123).
#include "common.h"

namespace {

struct AttnHeadArgs {
  const uint16_t* qkv;    // (3 * heads * D) fp16: q | k | v
  const uint16_t* qn_w;   // (heads * D) fp16
  const uint16_t* kn_w;   // (heads * D) fp16
  float eps;
  const uint16_t* cos_tab;  // (s_len, D) fp16
  const uint16_t* sin_tab;  // (s_len, D) fp16
  const int64_t* pos;       // device scalar
  int8_t* kc;
  uint16_t* ks;
  int8_t* vc;
  uint16_t* vs;
  int64_t code_head_stride;  // >= s_len * D
  int64_t s_len;
  int heads;
  float qk_scale;  // softmax scale * log2(e)
  uint16_t* out;   // (heads * D) fp16
};

// Sum over aligned groups of G lanes (G in {4, 8, 16}) with DPP row ops.
template <int G>
__device__ __forceinline__ float group_sum_dpp(float v) {
  v += dpp_f<LEMOQ_DPP_QUAD_1032>(v);
  v += dpp_f<LEMOQ_DPP_QUAD_2301>(v);
  if (G >= 8) v += dpp_f<LEMOQ_DPP_ROW_HALF_MIRROR>(v);
  if (G >= 16) v += dpp_f<LEMOQ_DPP_ROW_MIRROR>(v);
  return v;
}

template <int D>
struct HeadShape {
  static constexpr int LPT = D / 16;    // lanes per cached token row (16 codes per lane)
  static constexpr int TPW = 64 / LPT;  // tokens per wave load
  static constexpr int U = 8;           // wave loads per iteration
  static constexpr int BLK = TPW * U;   // tokens per wave iteration
  static constexpr int NW = 8;          // waves per block
  static constexpr int EPL = D / 64;    // prologue elements per lane
  static_assert(LPT == 4 || LPT == 8 || LPT == 16, "head_dim must be 64, 128 or 256");
};

template <int D>
struct TokBlock {
  u32x4 k[HeadShape<D>::U], v[HeadShape<D>::U];
  uint16_t ks[HeadShape<D>::U], vs[HeadShape<D>::U];
};

template <int D>
__device__ __forceinline__ void issue_tokens(TokBlock<D>& b, const int8_t* __restrict__ kb,
                                             const int8_t* __restrict__ vb,
                                             const uint16_t* __restrict__ ksh,
                                             const uint16_t* __restrict__ vsh, int64_t base,
                                             int64_t cap, int tl, int dl) {
  using S = HeadShape<D>;
#pragma unroll
  for (int u = 0; u < S::U; ++u) {
    int64_t t = base + u * S::TPW + tl;
    t = t < cap ? t : cap - 1;  // clamped: always a valid slot; validity is decided later
    b.k[u] = load_stream16(kb + t * D + dl * 16);
    b.v[u] = load_stream16(vb + t * D + dl * 16);
    b.ks[u] = ksh[t];
    b.vs[u] = vsh[t];
  }
}

struct SoftmaxState {
  float m, l;
  float acc[16];
};

// Online-softmax update with U token slices per lane (token base + u*TPW + tl),
// valid when below n; wave-uniform running max.
template <int D>
__device__ __forceinline__ void fold_tokens(SoftmaxState& st, const TokBlock<D>& b, const XChunk& qx,
                                            int64_t base, int64_t n, int tl, float qk_scale) {
  using S = HeadShape<D>;
  float sc[S::U];
  bool valid[S::U];
#pragma unroll
  for (int u = 0; u < S::U; ++u) {
    const int64_t t = base + u * S::TPW + tl;
    valid[u] = t < n;
    const float d = group_sum_dpp<S::LPT>(dot16_i8(b.k[u], qx, 0.0f));
    sc[u] = valid[u] ? (d * qk_scale) * h2f(b.ks[u]) : -INFINITY;
  }
  float mx = sc[0];
#pragma unroll
  for (int u = 1; u < S::U; ++u) mx = fmaxf(mx, sc[u]);
  mx = wave_max(mx);
  const float m_new = fmaxf(st.m, mx);
  if (m_new == -INFINITY) return;  // no valid token in this block (wave-uniform)
  const float alpha = exp2f(st.m - m_new);
  st.l *= alpha;
#pragma unroll
  for (int e = 0; e < 16; ++e) st.acc[e] *= alpha;
#pragma unroll
  for (int u = 0; u < S::U; ++u) {
    const float p = exp2f(sc[u] - m_new);  // 0 for invalid slices (sc = -inf)
    st.l += p;
    // an invalid slice may hold anything (its slot was read speculatively):
    // select, never multiply, so a NaN scale there cannot reach acc
    const float pw = valid[u] ? p * h2f(b.vs[u]) : 0.0f;
    const uint32_t w[4] = {b.v[u].x, b.v[u].y, b.v[u].z, b.v[u].w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        st.acc[4 * i + q] = fmaf(pw, (float)(int8_t)((w[i] >> (8 * q)) & 0xFFu), st.acc[4 * i + q]);
  }
  st.m = m_new;
}

template <int D>
__global__ __launch_bounds__(512) void attn_head_i8_kernel(const AttnHeadArgs a) {
  using S = HeadShape<D>;
  constexpr int LPT = S::LPT, TPW = S::TPW, BLK = S::BLK, NW = S::NW, EPL = S::EPL;
  __shared__ __align__(16) uint16_t q_s[D];
  __shared__ __align__(16) int8_t knew_s[D];
  __shared__ __align__(16) int8_t vnew_s[D];
  __shared__ float kvs_s[2];
  __shared__ float wm[NW], wl[NW];
  __shared__ float wacc[NW][D];

  const int h = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int dl = lane % LPT, tl = lane / LPT;
  const int HD = a.heads * D;
  const int64_t cap = a.s_len;
  const int8_t* kb = a.kc + (int64_t)h * a.code_head_stride;
  const int8_t* vb = a.vc + (int64_t)h * a.code_head_stride;
  const uint16_t* ksh = a.ks + (int64_t)h * cap;
  const uint16_t* vsh = a.vs + (int64_t)h * cap;

  // First block of cached tokens: issued before *pos arrives.
  TokBlock<D> tb;
  int64_t base = (int64_t)wave * BLK;
  issue_tokens<D>(tb, kb, vb, ksh, vsh, base, cap, tl, dl);

  const int64_t pos = a.pos[0];
  const bool pos_ok = pos >= 0 && pos < cap;
  const int64_t n_cache = pos_ok ? pos : 0;  // tokens [0, pos) come from the cache

  if (wave < 3) {
    // Prologue: wave 0 -> q, wave 1 -> new k (normed, rotated, quantised),
    // wave 2 -> new v (quantised).  Lane holds elements d0 .. d0+EPL-1 of head h.
    const int which = wave;
    const uint16_t* src = a.qkv + (int64_t)which * HD;
    const int d0 = lane * EPL;
    float o[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) o[i] = h2f(src[h * D + d0 + i]);
    if (which < 2) {
      const uint16_t* nw = which == 0 ? a.qn_w : a.kn_w;
      const int64_t prow = pos_ok ? pos : 0;
      float wv[EPL], cv[EPL], sv[EPL];
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        wv[i] = h2f(nw[h * D + d0 + i]);
        cv[i] = h2f(a.cos_tab[prow * D + d0 + i]);
        sv[i] = h2f(a.sin_tab[prow * D + d0 + i]);
      }
      float ssq = 0.0f;
      for (int i = lane * 8; i < HD; i += 64 * 8) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(src + i);
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float x0 = h2f((uint16_t)(w4[q] & 0xFFFFu)), x1 = h2f((uint16_t)(w4[q] >> 16));
          ssq = fmaf(x0, x0, ssq);
          ssq = fmaf(x1, x1, ssq);
        }
      }
      const float rstd = 1.0f / sqrtf(wave_sum(ssq) / (float)HD + a.eps);
      const bool first = lane < 32;  // d < D/2; the rotate_half partner is lane ^ 32
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        const float xn = h2f(f2h(h2f(f2h(o[i] * rstd)) * wv[i]));
        const float xs = __shfl_xor(xn, 32, 64);
        o[i] = h2f(f2h(first ? xn * cv[i] + (-xs) * sv[i] : xn * cv[i] + xs * sv[i]));
      }
    }
    if (which == 0) {
#pragma unroll
      for (int i = 0; i < EPL; ++i) q_s[d0 + i] = f2h(o[i]);
    } else {
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) amax = fmaxf(amax, fabsf(o[i]));
      amax = wave_max(amax);
      const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
      const uint16_t s16 = f2h(s);
      int8_t* lds = which == 1 ? knew_s : vnew_s;
      int8_t* dst = (which == 1 ? a.kc : a.vc) + (int64_t)h * a.code_head_stride + (pos_ok ? pos : 0) * D;
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        float qv = rintf(o[i] / s);
        qv = fminf(fmaxf(qv, -127.0f), 127.0f);
        const int8_t c = (int8_t)(int)qv;
        lds[d0 + i] = c;
        if (pos_ok) dst[d0 + i] = c;
      }
      if (lane == 0) {
        kvs_s[which - 1] = h2f(s16);
        if (pos_ok) (which == 1 ? a.ks : a.vs)[(int64_t)h * cap + pos] = s16;
      }
    }
  }
  __syncthreads();

  XChunk qx;
  load_xchunk(q_s + dl * 16, qx);
  SoftmaxState st;
  st.m = -INFINITY;
  st.l = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) st.acc[e] = 0.0f;

  for (bool first = true; base < n_cache; base += NW * BLK, first = false) {
    if (!first) issue_tokens<D>(tb, kb, vb, ksh, vsh, base, cap, tl, dl);
    LEMOQ_LOADS_ISSUED();
    fold_tokens<D>(st, tb, qx, base, n_cache, tl, a.qk_scale);
  }
  if (wave == 0 && pos_ok) {
    // The new token at slot pos, from LDS: only the lanes of token group 0 are valid.
    TokBlock<D> nb;
#pragma unroll
    for (int u = 0; u < S::U; ++u) {
      nb.k[u] = *reinterpret_cast<const u32x4*>(knew_s + dl * 16);
      nb.v[u] = *reinterpret_cast<const u32x4*>(vnew_s + dl * 16);
      nb.ks[u] = f2h(kvs_s[0]);
      nb.vs[u] = f2h(kvs_s[1]);
    }
    // token index of slice (u, tl) is u*TPW + tl: only (0, 0) is below 1.
    fold_tokens<D>(st, nb, qx, 0, 1, tl, a.qk_scale);
  }

  // Sum the token groups of the wave (lanes with the same slice dl).
#pragma unroll
  for (int o = LPT; o < 64; o <<= 1) {
    st.l += __shfl_xor(st.l, o, 64);
#pragma unroll
    for (int e = 0; e < 16; ++e) st.acc[e] += __shfl_xor(st.acc[e], o, 64);
  }
  if (lane == 0) {
    wm[wave] = st.m;
    wl[wave] = st.l;
  }
  if (tl == 0) {
#pragma unroll
    for (int e = 0; e < 16; ++e) wacc[wave][dl * 16 + e] = st.acc[e];
  }
  __syncthreads();
  for (int t = threadIdx.x; t < D; t += 64 * NW) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, wm[w]);
    float num = 0.0f, den = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float f = exp2f(wm[w] - M);
        num += wacc[w][t] * f;
        den += wl[w] * f;
      }
    }
    a.out[(int64_t)h * D + t] = f2h(den > 0.0f ? num / den : num);
  }
}

}  // namespace

extern "C" int lemoq_attn_decode_fused_i8(const uint16_t* qkv, int64_t heads, int64_t head_dim,
                                          const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                                          float eps, const uint16_t* cos_tab,
                                          const uint16_t* sin_tab, const int64_t* pos,
                                          int8_t* kc, uint16_t* ks, int8_t* vc, uint16_t* vs,
                                          int64_t code_head_stride, int64_t s_len, float qk_scale,
                                          uint16_t* out, void* stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !pos || !kc || !ks || !vc || !vs ||
      !out)
    return LEMOQ_ERR_NULL;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return LEMOQ_ERR_UNSUPPORTED;
  if (heads <= 0 || heads > 65535 || heads * head_dim > 65536) return LEMOQ_ERR_SHAPE;
  if (s_len <= 0 || code_head_stride < s_len * head_dim) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(qkv) || !lemoq_aligned16(kc) || !lemoq_aligned16(vc) ||
      code_head_stride % 16 != 0)
    return LEMOQ_ERR_ALIGN;
  AttnHeadArgs a;
  a.qkv = qkv;
  a.qn_w = q_norm_w;
  a.kn_w = k_norm_w;
  a.eps = eps;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.pos = pos;
  a.kc = kc;
  a.ks = ks;
  a.vc = vc;
  a.vs = vs;
  a.code_head_stride = code_head_stride;
  a.s_len = s_len;
  a.heads = (int)heads;
  a.qk_scale = qk_scale;
  a.out = out;
  hipStream_t st = lemoq_stream(stream);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL((attn_head_i8_kernel<64>), dim3((unsigned)heads), dim3(64 * HeadShape<64>::NW), 0, st, a); break;
    case 128: hipLaunchKernelGGL((attn_head_i8_kernel<128>), dim3((unsigned)heads), dim3(64 * HeadShape<64>::NW), 0, st, a); break;
    default: hipLaunchKernelGGL((attn_head_i8_kernel<256>), dim3((unsigned)heads), dim3(64 * HeadShape<64>::NW), 0, st, a); break;
  }
  LEMOQ_CHECK_LAUNCH();
}
