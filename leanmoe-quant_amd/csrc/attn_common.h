// Split-KV decode attention building blocks shared by the fused per-layer
// kernel (attn_fused.hip) and the standalone split kernels (attn.hip).
//
// A lane reads 16 bytes of a cached K or V row: 16 int8 codes (KV-INT8) or 8
// fp16 values.  A token row is LPT = D * bytes / 16 lanes, a wave load covers
// TPW = 64 / LPT tokens, and a wave token block is U loads (BLK = TPW * U
// tokens).  Token blocks are issued unconditionally, with slots at or beyond
// the split's end clamped to a valid slot and masked when folded, so a load
// never sits under a branch (the compiler would wait on it right away) and a
// slot past the filled length is never read.  The online softmax keeps a
// wave-uniform running max; INT8 rows fold the per-token scales
// (score = ((q.c) * qk_scale) * ks, acc += (p * vs) * c, l += p), which is
// the arithmetic of _attn_split_kernel_int8 / _attn_split_kernel
// (src/lemoq/kernels/_attn_triton.py:30-165 of the reference).
#pragma once

#include "common.h"

namespace lemoq_attn {

// Sum over aligned groups of G lanes (G in {4, 8, 16, 32}): DPP row ops, then
// the cross-row exchange for 32.
template <int G>
__device__ __forceinline__ float group_sum_lanes(float v, int lane) {
  static_assert(G == 4 || G == 8 || G == 16 || G == 32, "group of 4, 8, 16 or 32 lanes");
  v += dpp_f<LEMOQ_DPP_QUAD_1032>(v);
  v += dpp_f<LEMOQ_DPP_QUAD_2301>(v);
  if (G >= 8) v += dpp_f<LEMOQ_DPP_ROW_HALF_MIRROR>(v);
  if (G >= 16) v += dpp_f<LEMOQ_DPP_ROW_MIRROR>(v);
  if (G >= 32) v += xor16_get(v, lane);
  return v;
}

// Sum over the lanes that share lane % G (the 64 / G token groups of a wave).
template <int G>
__device__ __forceinline__ float groups_total(float v, int lane) {
  if constexpr (G == 32) {
    return v + xor32_get(v, lane);
  } else {
    return group_total<G>(v, lane);
  }
}

template <int D, bool I8, int U_>
struct TokShape {
  static constexpr bool INT8 = I8;
  static constexpr int EB = I8 ? 1 : 2;    // bytes per cached element
  static constexpr int EPL = 16 / EB;      // cached elements per lane load
  static constexpr int LPT = D / EPL;      // lanes per token row
  static constexpr int TPW = 64 / LPT;     // tokens per wave load
  static constexpr int U = U_;             // wave loads per token block
  static constexpr int BLK = TPW * U;      // tokens per wave token block
  static_assert(LPT == 4 || LPT == 8 || LPT == 16 || LPT == 32, "head_dim must be 64, 128 or 256");
};

template <class S>
struct TokBlock {
  u32x4 k[S::U], v[S::U];
  uint16_t ks[S::U], vs[S::U];  // per-token scales (KV-INT8 only)
};

// The lane's slice of q: 16 values in dot16_i8 order (int8 K) or 8 packed
// fp16 values (fp16 K).
template <bool I8>
struct QSlice;
template <>
struct QSlice<true> {
  XChunk x;
};
template <>
struct QSlice<false> {
  u32x4 x;
};

template <class S>
__device__ __forceinline__ void load_q(QSlice<S::INT8>& q, const uint16_t* qh, int dl) {
  if constexpr (S::INT8) {
    load_xchunk(qh + dl * 16, q.x);
  } else {
    q.x = *reinterpret_cast<const u32x4*>(qh + dl * 8);
  }
}

// Loads of the token block at `base` (token base + u*TPW + tl for load u);
// slots at or beyond `lim` are clamped to lim - 1 (a valid slot).
template <class S>
__device__ __forceinline__ void issue_tokens(TokBlock<S>& b, const uint8_t* __restrict__ kb,
                                             const uint8_t* __restrict__ vb,
                                             const uint16_t* __restrict__ ksh,
                                             const uint16_t* __restrict__ vsh, int64_t base,
                                             int64_t lim, int tl, int dl, int D) {
#pragma unroll
  for (int u = 0; u < S::U; ++u) {
    int64_t t = base + u * S::TPW + tl;
    t = t < lim ? t : lim - 1;
    const int64_t off = t * D * S::EB + dl * 16;
    b.k[u] = load_stream16(reinterpret_cast<const int8_t*>(kb + off));
    b.v[u] = load_stream16(reinterpret_cast<const int8_t*>(vb + off));
    if constexpr (S::INT8) {
      b.ks[u] = ksh[t];
      b.vs[u] = vsh[t];
    }
  }
}

template <int EPL>
struct SoftmaxState {
  float m, l;
  float acc[EPL];
};

template <int EPL>
__device__ __forceinline__ void softmax_init(SoftmaxState<EPL>& st) {
  st.m = -INFINITY;
  st.l = 0.0f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) st.acc[e] = 0.0f;
}

__device__ __forceinline__ float qk_dot_f16(const u32x4 k, const u32x4 q) {
  float a = __builtin_amdgcn_fdot2(as_h2(k.x), as_h2(q.x), 0.0f, false);
  a = __builtin_amdgcn_fdot2(as_h2(k.y), as_h2(q.y), a, false);
  a = __builtin_amdgcn_fdot2(as_h2(k.z), as_h2(q.z), a, false);
  return __builtin_amdgcn_fdot2(as_h2(k.w), as_h2(q.w), a, false);
}

// Online-softmax update with the token block at `base`; loads at or beyond
// `n` are masked (a masked slot may hold anything: its weight is selected to
// zero, never multiplied, so a NaN scale or value there cannot reach acc).
template <class S>
__device__ __forceinline__ void fold_tokens(SoftmaxState<S::EPL>& st, const TokBlock<S>& b,
                                            const QSlice<S::INT8>& q, int64_t base, int64_t n,
                                            int tl, int lane, float qk_scale) {
  float sc[S::U];
  bool valid[S::U];
#pragma unroll
  for (int u = 0; u < S::U; ++u) {
    const int64_t t = base + u * S::TPW + tl;
    valid[u] = t < n;
    float d;
    if constexpr (S::INT8) {
      d = group_sum_lanes<S::LPT>(dot16_i8(b.k[u], q.x, 0.0f), lane);
      sc[u] = valid[u] ? (d * qk_scale) * h2f(b.ks[u]) : -INFINITY;
    } else {
      d = group_sum_lanes<S::LPT>(qk_dot_f16(b.k[u], q.x), lane);
      sc[u] = valid[u] ? d * qk_scale : -INFINITY;
    }
  }
  float mx = sc[0];
#pragma unroll
  for (int u = 1; u < S::U; ++u) mx = fmaxf(mx, sc[u]);
  mx = wave_max(mx);
  const float m_new = fmaxf(st.m, mx);
  // No valid token so far (m_new == -inf, wave-uniform): fold against 0
  // instead, which keeps the state at (m = -inf, l = 0, acc = 0) -- what an
  // early return would keep -- without a branch (at the join of a branch the
  // compiler waits for every load in flight, the token blocks ahead included).
  const float m_ref = m_new == -INFINITY ? 0.0f : m_new;
  const float alpha = exp2f(st.m - m_ref);
  st.l *= alpha;
#pragma unroll
  for (int e = 0; e < S::EPL; ++e) st.acc[e] *= alpha;
#pragma unroll
  for (int u = 0; u < S::U; ++u) {
    const float p = exp2f(sc[u] - m_ref);  // 0 for masked loads (sc = -inf)
    st.l += p;
    const uint32_t w[4] = {b.v[u].x, b.v[u].y, b.v[u].z, b.v[u].w};
    if constexpr (S::INT8) {
      const float pw = valid[u] ? p * h2f(b.vs[u]) : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k)
          st.acc[4 * i + k] = fmaf(pw, (float)(int8_t)((w[i] >> (8 * k)) & 0xFFu), st.acc[4 * i + k]);
    } else {
      const float pw = valid[u] ? p : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        st.acc[2 * i] = fmaf(pw, valid[u] ? h2f((uint16_t)(w[i] & 0xFFFFu)) : 0.0f, st.acc[2 * i]);
        st.acc[2 * i + 1] = fmaf(pw, valid[u] ? h2f((uint16_t)(w[i] >> 16)) : 0.0f, st.acc[2 * i + 1]);
      }
    }
  }
  st.m = m_new;
}

// Pair sums across lane halves (gfx950 v_permlane32_swap) and across the rows
// of each half (v_permlane16_swap), for two values x, y per lane: lanes 0-31
// get x + x of lane ^ 32 and lanes 32-63 get y + y of lane ^ 32 (rows: even
// rows x, odd rows y, partner lane ^ 16).  One swap exchanges both: lanes 0-31
// receive the partner's x, lanes 32-63 the partner's y.  The lane's own value
// and the partner's are selected by lane and added, as in xor16_get /
// xor32_get: adding the swap's two results directly is miscompiled (the
// compiler adds the first result to itself).
__device__ __forceinline__ float halves_pair_sum(float x, float y, int lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, y), false, false);
  const bool lo = lane < 32;
  return (lo ? x : y) + __builtin_bit_cast(float, lo ? r[1] : r[0]);
}
__device__ __forceinline__ float rows_pair_sum(float x, float y, int lane) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, y), false, false);
  const bool even = (lane & 16) == 0;
  return (even ? x : y) + __builtin_bit_cast(float, even ? r[1] : r[0]);
}

// End of a split block: sum the token groups of each wave (the running max is
// wave-uniform), merge the NW wave states through LDS in wave order, and
// write the block's (m, l, acc[D]) partial; m = -inf for an empty split
// (l = 0, acc = 0).  wm/wl hold NW floats, wacc NW * D.
//
// The EPL accumulators of a lane are summed over its token group (the lanes
// sharing lane % LPT, partners lane ^ LPT, ^ 2 LPT, ... ^ 32) as a reduce-
// scatter: the pair sum across halves keeps elements [0, EPL/2) in the lower
// half and [EPL/2, EPL) in the upper, the pair sum across rows halves them
// again (LPT <= 16), and row rotations (LPT 4, 8) finish the sum.  A lane ends
// with V = EPL / 2 (or 4) fully summed elements instead of all EPL, and one
// lane of each group of duplicates writes them to LDS.
template <class S, int NW, int D>
__device__ __forceinline__ void finish_split(SoftmaxState<S::EPL>& st, float* wm, float* wl,
                                             float* wacc, int lane, int wave, int tl, int dl,
                                             int64_t pidx, float* __restrict__ m_out,
                                             float* __restrict__ l_out,
                                             float* __restrict__ acc_out) {
  constexpr int G = S::LPT, E = S::EPL;
  constexpr bool X16 = G <= 16;            // the row pair is a partner too
  constexpr int V = X16 ? E / 4 : E / 2;   // elements per lane after the scatter
  static_assert(G <= 32 && V >= 1, "token groups of 4, 8, 16 or 32 lanes");
  st.l = groups_total<G>(st.l, lane);
  float h[E / 2];
#pragma unroll
  for (int i = 0; i < E / 2; ++i) h[i] = halves_pair_sum(st.acc[i], st.acc[i + E / 2], lane);
  float v[V];
  if constexpr (X16) {
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = rows_pair_sum(h[i], h[i + V], lane);
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = h[i];
  }
#pragma unroll
  for (int i = 0; i < V; ++i) {
    if (G == 4) v[i] += dpp_f<LEMOQ_DPP_ROW_ROR4>(v[i]);
    if (G <= 8) v[i] += dpp_f<LEMOQ_DPP_ROW_ROR8>(v[i]);
  }
  if (lane == 0) {
    wm[wave] = st.m;
    wl[wave] = st.l;
  }
  // lanes whose in-row token bits are zero hold distinct element ranges
  if (G > 16 || (lane & 15) < G) {
    const int base = ((lane & 32) ? E / 2 : 0) + ((X16 && (lane & 16)) ? E / 4 : 0);
    float* dst = wacc + wave * D + dl * E + base;
#pragma unroll
    for (int i = 0; i < V; ++i) dst[i] = v[i];
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
        num += wacc[w * D + t] * f;
        den += wl[w] * f;
      }
    }
    acc_out[pidx * D + t] = num;
    if (t == 0) {
      m_out[pidx] = M;
      l_out[pidx] = den;
    }
  }
}

// LSE merge of the NS split partials of one head by one wave (the merge of
// _attn_merge_kernel, src/lemoq/kernels/_attn_triton.py of the reference).
// Lane j < NS holds split j's running max m_j and sum l_j (other lanes any
// valid value).  Returns w_j = 2^(m_j - M) in lane j (0 for j >= NS) and sets
// den = sum_j l_j w_j (wave-uniform), M = max_j m_j, or 0 when every split is
// empty.
__device__ __forceinline__ float lse_weight(float mraw, float lraw, int lane, int NS, float& den) {
  const float mj = lane < NS ? mraw : -INFINITY;  // selects, not branches
  const float lj = lane < NS ? lraw : 0.0f;
  float M = wave_max(mj);
  if (!(M > -INFINITY)) M = 0.0f;  // every split empty: out = 0
  const float wj = exp2f(mj - M);
  den = wave_sum(lj * wj);
  return wj;
}

// fp16(num / den) with num = sum_j a[j] w_j in split order (w_j read from
// lane j; slots j >= NS carry weight 0 and add exactly nothing).
template <int NSMAX>
__device__ __forceinline__ uint16_t lse_out(const float (&a)[NSMAX], float wj, float den) {
  float num = 0.0f;
#pragma unroll
  for (int j = 0; j < NSMAX; ++j) num += a[j] * lane_f(wj, j);
  return f2h(den > 0.0f ? num / den : num);
}

}  // namespace lemoq_attn
