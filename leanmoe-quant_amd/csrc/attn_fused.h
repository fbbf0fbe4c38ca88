// The split-KV block of the fused per-layer attention over the KV-INT8 or the
// fp16 cache (q_norm/k_norm, RoPE, the cache write of the new token, online
// softmax over the block's cached tokens), launched by attn_fused.hip.
//
// attn_split_fused_i8 / _f16: grid (num_splits, heads), 4 waves per block.  Block
// (s, h) covers tokens [s*c, min((s+1)*c, n)) of head h with n = *pos + 1 and
// c = ceil(n / num_splits) (the reference's split rule,
// src/lemoq/kernels/attn_decode.py:295-354), and does in one launch what the
// reference does in four (attn_decode.py:882-1000):
//   - q_norm over all heads*D values of q (HF rounding points) and RoPE at
//     *pos for head h (wave 0, every block: the 4 KB row is L2-resident);
//   - in the one block whose range holds *pos: k_norm + RoPE of the new k and
//     the cache write of the new k and v rows (waves 1 and 2): their KV-INT8
//     quantisation, or the fp16 rows as they are (the reference's
//     kv_direct_write, src/lemoq/kernels/kv_direct.py:110-137, when KV-INT8
//     is off), written to slot *pos of the cache and kept in LDS;
//   - the online softmax over its cached tokens, for KV-INT8 with the
//     per-token scales folded in (score = ((q.c) * qk_scale) * ks,
//     acc += (p * vs) * c, l += p), the new token folded from LDS (never read
//     back from the slot just written), and the block's (m, l, acc[D])
//     partial.
// The LSE merge of the partials is lemoq_attn_merge.  Each wave keeps two
// blocks of token loads in flight (double buffering); the token groups of a
// wave are summed with DPP row rotations and the gfx950 cross-row swaps.
//
// Arithmetic restates _attn_split_kernel_int8
// (src/lemoq/kernels/_attn_triton.py:102-165) and, for fp16 rows,
// _attn_split_kernel (:30-99), the KV write
// (src/lemoq/kernels/kv_int8.py:196-216), _rope_one_kernel
// (src/lemoq/kernels/rope.py:101-123) and the HF q_norm/k_norm RMSNorm.
#pragma once

#include "attn_common.h"

namespace lemoq_attn_fused {

struct AttnSplitArgs {
  const uint16_t* qkv;    // (3 * heads * D) fp16: q | k | v
  const uint16_t* qn_w;   // (heads * D) fp16
  const uint16_t* kn_w;   // (heads * D) fp16
  float eps;
  const uint16_t* cos_tab;  // (s_len, D) fp16
  const uint16_t* sin_tab;  // (s_len, D) fp16
  const int64_t* pos;       // device scalar
  void* kc;                 // (heads, code_head_stride) int8 codes, or fp16 rows
  uint16_t* ks;             // (heads, s_len) fp16 scales (KV-INT8 only)
  void* vc;
  uint16_t* vs;
  int64_t code_head_stride;  // elements, >= s_len * D
  int64_t s_len;
  int heads;
  int ns;
  float qk_scale;  // softmax scale * log2(e)
  float clip;      // clip_qkv bound (+inf: none)
  float* m_out;    // (heads, ns)
  float* l_out;    // (heads, ns)
  float* acc_out;  // (heads, ns, D)
};

template <int D, bool I8, int NW_ = 8, int U_ = 4>
struct HeadShape {
  using T = lemoq_attn::TokShape<D, I8, U_>;  // KV-INT8 or fp16 token rows
  static constexpr int LPT = T::LPT;    // lanes per cached token row (16 bytes per lane)
  static constexpr int BLK = T::BLK;    // tokens per wave token block
  static constexpr int NW = NW_;        // waves per block
  static constexpr int EPL = D / 64;    // prologue elements per lane
  static_assert(NW >= 3, "waves 0..2 carry the q and new k/v prologue");
};

// LDS of one split block (the new k / v rows as the cache holds them: EB
// bytes per element).
template <int D, int NW, int EB>
struct AttnFusedSmem {
  alignas(16) uint16_t q_s[D];
  alignas(16) uint8_t knew_s[D * EB];
  alignas(16) uint8_t vnew_s[D * EB];
  float kvs_s[2];
  float wm[NW], wl[NW];
  float wacc[NW * D];
};

template <int D, bool I8, int NW_, int U_>
__device__ __forceinline__ void attn_split_fused_block(const AttnSplitArgs& a, int sp, int h,
                                                       AttnFusedSmem<D, NW_, I8 ? 1 : 2>& sm) {
  using S = HeadShape<D, I8, NW_, U_>;
  using T = typename S::T;
  constexpr int BLK = S::BLK, NW = S::NW, EPL = S::EPL, EB = T::EB;
  constexpr int STRIDE = NW * BLK;
  uint16_t* q_s = sm.q_s;
  uint8_t* knew_s = sm.knew_s;
  uint8_t* vnew_s = sm.vnew_s;
  float* kvs_s = sm.kvs_s;
  float* wm = sm.wm;
  float* wl = sm.wl;
  float* wacc = sm.wacc;

  // wave from a scalar register: the branches on it below are scalar branches
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int dl = lane % T::LPT, tl = lane / T::LPT;
  const int HD = a.heads * D;
  const int64_t cap = a.s_len;
  const uint8_t* kb = static_cast<const uint8_t*>(a.kc) + (int64_t)h * a.code_head_stride * EB;
  const uint8_t* vb = static_cast<const uint8_t*>(a.vc) + (int64_t)h * a.code_head_stride * EB;
  const uint16_t* ksh = I8 ? a.ks + (int64_t)h * cap : nullptr;  // read only for KV-INT8
  const uint16_t* vsh = I8 ? a.vs + (int64_t)h * cap : nullptr;

  const int64_t pos = a.pos[0];  // a scalar load, issued first

  // Issue order.  The vector loads of a wave retire in issue order, so what
  // is needed first is issued first: the prologue rows that do not depend on
  // *pos (q, or the new k / v, and the norm weights) go out before *pos has
  // arrived; then the cos/sin row at *pos; then the first token block.  The
  // q norm thus overlaps the token loads instead of waiting behind them.
  // Waves 1 and 2 load the new k / v rows in every block (only the block that
  // holds *pos uses them: *pos is not known yet).
  constexpr int QV = 8;  // 16-byte row slices per lane held in registers (rows <= 4096)
  const bool pro_wave = wave < 3;
  const int which = wave;
  const uint16_t* src = a.qkv + (int64_t)which * HD;
  // 16-bit values held one per 32-bit register: packing two into one register
  // would make the compiler wait for both loads inside the branch.
  uint32_t ob[EPL], wb[EPL], cb[EPL], sb[EPL];
  u32x4 qrow[QV];
  if (pro_wave) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) ob[i] = src[h * D + lane + 64 * i];
    if (which < 2) {
      const uint16_t* nw = which == 0 ? a.qn_w : a.kn_w;
#pragma unroll
      for (int j = 0; j < QV; ++j) {
        const int i = lane * 8 + j * 64 * 8;
        qrow[j] = *reinterpret_cast<const u32x4*>(src + (i < HD ? i : 0));  // masked below
      }
#pragma unroll
      for (int i = 0; i < EPL; ++i) wb[i] = nw[h * D + lane + 64 * i];
    }
  }

  // (cap < 2^31, checked on the host: the split arithmetic is 32-bit.)
  const bool pos_ok = pos >= 0 && pos < cap;
  const uint32_t n_tot = pos_ok ? (uint32_t)pos + 1u : 0u;  // attention over tokens [0, pos]
  const uint32_t chunk = (n_tot + (uint32_t)a.ns - 1u) / (uint32_t)a.ns;
  const int64_t start = (int64_t)sp * chunk;
  const int64_t end = start + chunk < n_tot ? start + chunk : (int64_t)n_tot;
  const bool owns_new = pos_ok && start <= pos && pos < end;
  const int64_t cend = owns_new ? pos : end;  // cached tokens [start, cend)

  if (pro_wave && which < 2) {
    const int64_t prow = pos_ok ? pos : 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      cb[i] = a.cos_tab[prow * D + lane + 64 * i];
      sb[i] = a.sin_tab[prow * D + lane + 64 * i];
    }
  }
  // The first token block is issued unconditionally (slots clamped into
  // [0, max(cend, 1)), folds masked by cend): a load under a branch lets the
  // compiler unpack its bytes right after the issue, which would wait on it
  // before the prologue below could overlap it.
  lemoq_attn::TokBlock<T> ta, tb;
  int64_t base = start + (int64_t)wave * BLK;
  const int64_t lim = cend > 0 ? cend : 1;
  lemoq_attn::issue_tokens<T>(ta, kb, vb, ksh, vsh, base, lim, tl, dl, D);
  LEMOQ_LOADS_ISSUED();

  if (wave == 0 || (owns_new && wave < 3)) {
    // Prologue: wave 0 -> q (every block), wave 1 -> new k (normed, rotated,
    // quantised), wave 2 -> new v (quantised).  Element i of a lane is
    // d = lane + 64 i, so for D >= 128 a lane holds both rotate_half partners
    // (d and d + D/2) and RoPE needs no cross-lane exchange; for D = 64 the
    // partner is lane ^ 32.
    const float clip16 = h2f(f2h(a.clip));
    float o[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) o[i] = h2f(ob[i]);
    if (which == 2) {
#pragma unroll
      for (int i = 0; i < EPL; ++i) o[i] = clip_qkv(o[i], a.clip, clip16);
    }
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
      for (int i = 0; i < EPL; ++i)
        xn[i] = clip_qkv(h2f(f2h(h2f(f2h(o[i] * rstd)) * h2f(wb[i]))), a.clip, clip16);
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
    } else if constexpr (!I8) {
      // fp16 cache: the rotated k / the (clipped) v row as it is
      uint16_t* lds = reinterpret_cast<uint16_t*>(which == 1 ? knew_s : vnew_s);
      uint16_t* dst = static_cast<uint16_t*>(which == 1 ? a.kc : a.vc) + (int64_t)h * a.code_head_stride +
                      pos * D;
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        const uint16_t b = f2h(o[i]);
        lds[lane + 64 * i] = b;
        dst[lane + 64 * i] = b;
      }
    } else {
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) amax = fmaxf(amax, fabsf(o[i]));
      amax = wave_max(amax);
      const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
      const uint16_t s16 = f2h(s);
      int8_t* lds = reinterpret_cast<int8_t*>(which == 1 ? knew_s : vnew_s);
      int8_t* dst = static_cast<int8_t*>(which == 1 ? a.kc : a.vc) + (int64_t)h * a.code_head_stride + pos * D;
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

  lemoq_attn::QSlice<I8> qx;
  lemoq_attn::load_q<T>(qx, q_s, dl);
  lemoq_attn::SoftmaxState<T::EPL> st;
  lemoq_attn::softmax_init(st);

  // Two token blocks in flight: fold one while the next one loads.  The next
  // block is issued only when the wave has one (a wave-uniform branch): a
  // load of nothing would still have to retire before the block's closing
  // barrier.
  while (base < cend) {
    int64_t nb = base + STRIDE;
    bool more = nb < cend;
    if (more) lemoq_attn::issue_tokens<T>(tb, kb, vb, ksh, vsh, nb, lim, tl, dl, D);
    LEMOQ_LOADS_ISSUED();
    lemoq_attn::fold_tokens<T>(st, ta, qx, base, cend, tl, lane, a.qk_scale);
    if (!more) break;
    base = nb;
    nb = base + STRIDE;
    more = nb < cend;
    if (more) lemoq_attn::issue_tokens<T>(ta, kb, vb, ksh, vsh, nb, lim, tl, dl, D);
    LEMOQ_LOADS_ISSUED();
    lemoq_attn::fold_tokens<T>(st, tb, qx, base, cend, tl, lane, a.qk_scale);
    if (!more) break;
    base = nb;
  }
  if (wave == NW - 1 && owns_new) {
    // The new token at slot pos, from LDS: only slice (u = 0, tl = 0) is
    // valid.  The last wave holds the fewest cached tokens of the split.
    lemoq_attn::TokBlock<T> nbk;
#pragma unroll
    for (int u = 0; u < T::U; ++u) {
      nbk.k[u] = *reinterpret_cast<const u32x4*>(knew_s + dl * 16);
      nbk.v[u] = *reinterpret_cast<const u32x4*>(vnew_s + dl * 16);
      if constexpr (I8) {
        nbk.ks[u] = f2h(kvs_s[0]);
        nbk.vs[u] = f2h(kvs_s[1]);
      }
    }
    lemoq_attn::fold_tokens<T>(st, nbk, qx, 0, 1, tl, lane, a.qk_scale);
  }
  lemoq_attn::finish_split<T, NW, D>(st, wm, wl, wacc, lane, wave, tl, dl,
                                               (int64_t)h * a.ns + sp, a.m_out, a.l_out, a.acc_out);
}

}  // namespace lemoq_attn_fused
