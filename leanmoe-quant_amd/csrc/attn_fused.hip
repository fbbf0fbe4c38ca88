// Fused per-layer attention of the decode step over the KV-INT8 cache.
//
// attn_split_fused_i8: grid (num_splits, heads), 4 waves per block.  Block
// (s, h) covers tokens [s*c, min((s+1)*c, n)) of head h with n = *pos + 1 and
// c = ceil(n / num_splits) (the reference's split rule,
// src/lemoq/kernels/attn_decode.py:295-354), and does in one launch what the
// reference does in four (attn_decode.py:882-1000):
//   - q_norm over all heads*D values of q (HF rounding points) and RoPE at
//     *pos for head h (wave 0, every block: the 4 KB row is L2-resident);
//   - in the one block whose range holds *pos: k_norm + RoPE of the new k and
//     the KV-INT8 quantisation of the new k and v rows (waves 1 and 2),
//     written to slot *pos of the cache and kept in LDS;
//   - the online softmax over its cached tokens with the per-token scales
//     folded in (score = ((q.c) * qk_scale) * ks, acc += (p * vs) * c,
//     l += p), the new token folded from LDS (never read back from the slot
//     just written), and the block's (m, l, acc[D]) partial.
// The LSE merge of the partials is lemoq_attn_merge.  Each wave keeps two
// blocks of token loads in flight (double buffering); the token groups of a
// wave are summed with DPP row rotations and the gfx950 cross-row swaps.
//
// Arithmetic restates _attn_split_kernel_int8
// (src/lemoq/kernels/_attn_triton.py:102-165), the KV write
// (src/lemoq/kernels/kv_int8.py:196-216), _rope_one_kernel
// (src/lemoq/kernels/rope.py:101-123) and the HF q_norm/k_norm RMSNorm.
#include "common.h"

namespace {

struct AttnSplitArgs {
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
  int ns;
  float qk_scale;  // softmax scale * log2(e)
  float* m_out;    // (heads, ns)
  float* l_out;    // (heads, ns)
  float* acc_out;  // (heads, ns, D)
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

template <int D, int NW_ = 8, int U_ = 4>
struct HeadShape {
  static constexpr int LPT = D / 16;    // lanes per cached token row (16 codes per lane)
  static constexpr int TPW = 64 / LPT;  // tokens per wave load
  static constexpr int U = U_;          // wave loads per token block
  static constexpr int BLK = TPW * U;   // tokens per wave token block
  static constexpr int NW = NW_;        // waves per block
  static constexpr int EPL = D / 64;    // prologue elements per lane
  static_assert(LPT == 4 || LPT == 8 || LPT == 16, "head_dim must be 64, 128 or 256");
  static_assert(NW >= 3, "waves 0..2 carry the q and new k/v prologue");
};

template <class S>
struct TokBlock {
  u32x4 k[S::U], v[S::U];
  uint16_t ks[S::U], vs[S::U];
};

// Loads of the token block at `base` (token base + u*TPW + tl for slice u);
// slots at or beyond `lim` are clamped to lim - 1 (a valid slot) and masked
// when folded.
template <int D, class S>
__device__ __forceinline__ void issue_tokens(TokBlock<S>& b, const int8_t* __restrict__ kb,
                                             const int8_t* __restrict__ vb,
                                             const uint16_t* __restrict__ ksh,
                                             const uint16_t* __restrict__ vsh, int64_t base,
                                             int64_t lim, int tl, int dl) {
#pragma unroll
  for (int u = 0; u < S::U; ++u) {
    int64_t t = base + u * S::TPW + tl;
    t = t < lim ? t : lim - 1;
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

// Online-softmax update with the token block at `base`; slices at or beyond
// `n` are masked.  The running max is wave-uniform.
template <class S>
__device__ __forceinline__ void fold_tokens(SoftmaxState& st, const TokBlock<S>& b, const XChunk& qx,
                                            int64_t base, int64_t n, int tl, float qk_scale) {
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
    const float p = exp2f(sc[u] - m_new);  // 0 for masked slices (sc = -inf)
    st.l += p;
    // a masked slice may hold anything (clamped slot): select, never multiply,
    // so a NaN scale there cannot reach acc
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

template <int D, int NW_ = 8, int U_ = 4>
__global__ __launch_bounds__(64 * NW_) void attn_split_fused_i8_kernel(const AttnSplitArgs a) {
  using S = HeadShape<D, NW_, U_>;
  constexpr int LPT = S::LPT, BLK = S::BLK, NW = S::NW, EPL = S::EPL;
  constexpr int STRIDE = NW * BLK;
  __shared__ __align__(16) uint16_t q_s[D];
  __shared__ __align__(16) int8_t knew_s[D];
  __shared__ __align__(16) int8_t vnew_s[D];
  __shared__ float kvs_s[2];
  __shared__ float wm[NW], wl[NW];
  __shared__ float wacc[NW][D];

  const int sp = blockIdx.x, h = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int dl = lane % LPT, tl = lane / LPT;
  const int HD = a.heads * D;
  const int64_t cap = a.s_len;
  const int8_t* kb = a.kc + (int64_t)h * a.code_head_stride;
  const int8_t* vb = a.vc + (int64_t)h * a.code_head_stride;
  const uint16_t* ksh = a.ks + (int64_t)h * cap;
  const uint16_t* vsh = a.vs + (int64_t)h * cap;

  const int64_t pos = a.pos[0];
  const bool pos_ok = pos >= 0 && pos < cap;
  const int64_t n_tot = pos_ok ? pos + 1 : 0;  // attention over tokens [0, pos]
  const int64_t chunk = (n_tot + a.ns - 1) / a.ns;
  const int64_t start = (int64_t)sp * chunk;
  const int64_t end = start + chunk < n_tot ? start + chunk : n_tot;
  const bool owns_new = pos_ok && start <= pos && pos < end;
  const int64_t cend = owns_new ? pos : end;  // cached tokens [start, cend)

  // The first token block is issued unconditionally (slots clamped into
  // [0, max(cend, 1)), folds masked by cend): a load under a branch lets the
  // compiler unpack its bytes right after the issue, which waits on it before
  // the prologue below could overlap it.
  TokBlock<S> ta, tb;
  int64_t base = start + (int64_t)wave * BLK;
  const int64_t lim = cend > 0 ? cend : 1;
  issue_tokens<D, S>(ta, kb, vb, ksh, vsh, base, lim, tl, dl);

  if (wave == 0 || (owns_new && wave < 3)) {
    // Prologue: wave 0 -> q (every block), wave 1 -> new k (normed, rotated,
    // quantised), wave 2 -> new v (quantised).  Element i of a lane is
    // d = lane + 64 i, so for D >= 128 a lane holds both rotate_half partners
    // (d and d + D/2) and RoPE needs no cross-lane exchange; for D = 64 the
    // partner is lane ^ 32.  Every prologue load (the lane's values, norm
    // weight, cos/sin row, and the whole q or k row for the sum of squares)
    // is issued as raw bits before any of them is used, so the prologue waits
    // on memory once.
    constexpr int QV = 8;  // 16-byte row slices per lane held in registers (rows <= 4096)
    const int which = wave;
    const uint16_t* src = a.qkv + (int64_t)which * HD;
    uint16_t ob[EPL], wb[EPL], cb[EPL], sb[EPL];
    u32x4 qrow[QV];
#pragma unroll
    for (int i = 0; i < EPL; ++i) ob[i] = src[h * D + lane + 64 * i];
    if (which < 2) {
      const uint16_t* nw = which == 0 ? a.qn_w : a.kn_w;
      const int64_t prow = pos_ok ? pos : 0;
#pragma unroll
      for (int j = 0; j < QV; ++j) {
        const int i = lane * 8 + j * 64 * 8;
        qrow[j] = *reinterpret_cast<const u32x4*>(src + (i < HD ? i : 0));  // masked below
      }
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        wb[i] = nw[h * D + lane + 64 * i];
        cb[i] = a.cos_tab[prow * D + lane + 64 * i];
        sb[i] = a.sin_tab[prow * D + lane + 64 * i];
      }
    }
    LEMOQ_LOADS_ISSUED();
    float o[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) o[i] = h2f(ob[i]);
    if (which < 2) {
      // Same sum-of-squares order as lemoq_qk_norm_rope_kv_i8 (slices
      // lane*8 + 512 j, ssq_f16x8), so both write identical KV bytes.
      float ssq = 0.0f;
#pragma unroll
      for (int j = 0; j < QV; ++j)
        if (lane * 8 + j * 64 * 8 < HD) ssq = ssq_f16x8(qrow[j], ssq);
      for (int i = lane * 8 + QV * 64 * 8; i < HD; i += 64 * 8)  // rows beyond 4096 values
        ssq = ssq_f16x8(*reinterpret_cast<const u32x4*>(src + i), ssq);
      const float rstd = 1.0f / sqrtf(wave_sum(ssq) / (float)HD + a.eps);
      float xn[EPL];
#pragma unroll
      for (int i = 0; i < EPL; ++i) xn[i] = h2f(f2h(h2f(f2h(o[i] * rstd)) * h2f(wb[i])));
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        const bool first = EPL == 1 ? lane < 32 : i < EPL / 2;  // d < D/2
        const float xs = EPL == 1 ? xor32_get(xn[i], lane) : xn[i ^ (EPL / 2)];
        const float cv = h2f(cb[i]), sv = h2f(sb[i]);
        o[i] = h2f(f2h(first ? xn[i] * cv + (-xs) * sv : xn[i] * cv + xs * sv));
      }
    }
    if (which == 0) {
#pragma unroll
      for (int i = 0; i < EPL; ++i) q_s[lane + 64 * i] = f2h(o[i]);
    } else {
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) amax = fmaxf(amax, fabsf(o[i]));
      amax = wave_max(amax);
      const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
      const uint16_t s16 = f2h(s);
      int8_t* lds = which == 1 ? knew_s : vnew_s;
      int8_t* dst = (which == 1 ? a.kc : a.vc) + (int64_t)h * a.code_head_stride + pos * D;
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        float qv = rintf(o[i] / s);
        qv = fminf(fmaxf(qv, -127.0f), 127.0f);
        const int8_t c = (int8_t)(int)qv;
        lds[lane + 64 * i] = c;
        dst[lane + 64 * i] = c;
      }
      if (lane == 0) {
        kvs_s[which - 1] = h2f(s16);
        (which == 1 ? a.ks : a.vs)[(int64_t)h * cap + pos] = s16;
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

  // Two token blocks in flight: fold one while the next one loads.  The
  // next block is issued unconditionally (clamped; at the end it re-reads
  // the split's last slot, an L2 hit) for the reason given above.
  while (base < cend) {
    int64_t nb = base + STRIDE;
    issue_tokens<D, S>(tb, kb, vb, ksh, vsh, nb, lim, tl, dl);
    LEMOQ_LOADS_ISSUED();
    fold_tokens<S>(st, ta, qx, base, cend, tl, a.qk_scale);
    base = nb;
    if (base >= cend) break;
    nb = base + STRIDE;
    issue_tokens<D, S>(ta, kb, vb, ksh, vsh, nb, lim, tl, dl);
    LEMOQ_LOADS_ISSUED();
    fold_tokens<S>(st, tb, qx, base, cend, tl, a.qk_scale);
    base = nb;
  }
  if (wave == NW - 1 && owns_new) {
    // The new token at slot pos, from LDS: only slice (u = 0, tl = 0) is
    // valid.  The last wave holds the fewest cached tokens of the split.
    TokBlock<S> nbk;
#pragma unroll
    for (int u = 0; u < S::U; ++u) {
      nbk.k[u] = *reinterpret_cast<const u32x4*>(knew_s + dl * 16);
      nbk.v[u] = *reinterpret_cast<const u32x4*>(vnew_s + dl * 16);
      nbk.ks[u] = f2h(kvs_s[0]);
      nbk.vs[u] = f2h(kvs_s[1]);
    }
    fold_tokens<S>(st, nbk, qx, 0, 1, tl, a.qk_scale);
  }

  // Sum the token groups of the wave (lanes with the same slice dl); the
  // running max is wave-uniform, so no rescale is needed.
  st.l = group_total<LPT>(st.l, lane);
#pragma unroll
  for (int e = 0; e < 16; ++e) st.acc[e] = group_total<LPT>(st.acc[e], lane);
  if (lane == 0) {
    wm[wave] = st.m;
    wl[wave] = st.l;
  }
  if (tl == 0) {
#pragma unroll
    for (int e = 0; e < 16; ++e) wacc[wave][dl * 16 + e] = st.acc[e];
  }
  __syncthreads();
  const int64_t pidx = (int64_t)h * a.ns + sp;
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
    a.acc_out[pidx * D + t] = num;
    if (t == 0) {
      a.m_out[pidx] = M;  // -inf for an empty split (l = 0, acc = 0)
      a.l_out[pidx] = den;
    }
  }
}

}  // namespace

extern "C" int lemoq_attn_split_fused_i8(const uint16_t* qkv, int64_t heads, int64_t head_dim,
                                         const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                                         float eps, const uint16_t* cos_tab,
                                         const uint16_t* sin_tab, const int64_t* pos, int8_t* kc,
                                         uint16_t* ks, int8_t* vc, uint16_t* vs,
                                         int64_t code_head_stride, int64_t s_len,
                                         int64_t num_splits, float qk_scale, float* m, float* l,
                                         float* acc, void* stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !pos || !kc || !ks || !vc || !vs ||
      !m || !l || !acc)
    return LEMOQ_ERR_NULL;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return LEMOQ_ERR_UNSUPPORTED;
  if (heads <= 0 || heads > 65535 || heads * head_dim > 65536) return LEMOQ_ERR_SHAPE;
  if (num_splits <= 0 || num_splits > 65535) return LEMOQ_ERR_SHAPE;
  if (s_len <= 0 || code_head_stride < s_len * head_dim) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(qkv) || !lemoq_aligned16(kc) || !lemoq_aligned16(vc) ||
      code_head_stride % 16 != 0)
    return LEMOQ_ERR_ALIGN;
  AttnSplitArgs a;
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
  a.ns = (int)num_splits;
  a.qk_scale = qk_scale;
  a.m_out = m;
  a.l_out = l;
  a.acc_out = acc;
  hipStream_t st = lemoq_stream(stream);
  const dim3 grid((unsigned)num_splits, (unsigned)heads);
  // 4 waves per block (two blocks share a CU), 2 token loads per wave in
  // flight per token block: the fastest shape measured at 1 100 and 4 200
  // cache slots with 16 splits (against 8 and 16 waves, 1 and 4 loads).
  const dim3 block(64 * 4);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL((attn_split_fused_i8_kernel<64, 4, 2>), grid, block, 0, st, a); break;
    case 128: hipLaunchKernelGGL((attn_split_fused_i8_kernel<128, 4, 2>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((attn_split_fused_i8_kernel<256, 4, 2>), grid, block, 0, st, a); break;
  }
  LEMOQ_CHECK_LAUNCH();
}
