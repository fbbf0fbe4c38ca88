// Split-KV decode attention (flash-decoding) for batch 1, q_len 1, over fp16
// or KV-INT8 caches, and the log-sum-exp merge of the splits.
//
// Split kernel: grid (num_splits, heads), 4 waves.  Block (s, h) covers
// tokens [s*c, min((s+1)*c, n)) of head h with n = *filled (clamped to the
// cache) and c = ceil(n / num_splits) (the reference's split rule,
// src/lemoq/kernels/attn_decode.py:295-354).  Each wave walks its
// interleaved token blocks with two blocks of loads in flight, an online
// softmax with a wave-uniform running max, and KV-INT8 scales folded in
// (attn_common.h); the four wave states are merged through LDS in a fixed
// order.  Tokens at or beyond the filled length are never loaded, so
// whatever the cache holds there (NaN included) cannot leak in.
#include "attn_common.h"

namespace {

template <int D, bool I8>
struct SplitShape {
  static constexpr int NW = 4;             // waves per block
  using T = lemoq_attn::TokShape<D, I8, I8 ? 2 : 4>;  // 16 tokens per wave block at D = 128
};

template <int D, bool I8>
__global__ __launch_bounds__(256) void attn_split_kernel(
    const uint16_t* __restrict__ q, const void* __restrict__ kp, const uint16_t* __restrict__ ks,
    const void* __restrict__ vp, const uint16_t* __restrict__ vs, int64_t head_stride,
    int64_t s_len, int64_t max_len, const int32_t* __restrict__ filled, int NS, float qk_scale,
    float* __restrict__ m_out, float* __restrict__ l_out, float* __restrict__ acc_out) {
  using T = typename SplitShape<D, I8>::T;
  constexpr int NW = SplitShape<D, I8>::NW;
  constexpr int STRIDE = NW * T::BLK;
  __shared__ float wm[NW], wl[NW];
  __shared__ float wacc[NW * D];

  const int sp = blockIdx.x, h = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int dl = lane % T::LPT;  // which 16-byte slice of the row
  const int tl = lane / T::LPT;  // which token of the wave load

  // This lane's slice of q first: the load counter retires in order.
  lemoq_attn::QSlice<I8> qx;
  lemoq_attn::load_q<T>(qx, q + (int64_t)h * D, dl);

  int64_t n = filled[0];
  n = n < 0 ? 0 : (n > max_len ? max_len : n);
  const int64_t chunk = (n + NS - 1) / NS;
  const int64_t start = (int64_t)sp * chunk;
  const int64_t end = start + chunk < n ? start + chunk : n;

  const uint8_t* kb = reinterpret_cast<const uint8_t*>(kp) + (int64_t)h * head_stride * T::EB;
  const uint8_t* vb = reinterpret_cast<const uint8_t*>(vp) + (int64_t)h * head_stride * T::EB;
  const uint16_t* ksh = I8 ? ks + (int64_t)h * s_len : nullptr;
  const uint16_t* vsh = I8 ? vs + (int64_t)h * s_len : nullptr;

  lemoq_attn::TokBlock<T> ta, tb;
  int64_t base = start + (int64_t)wave * T::BLK;
  const int64_t lim = end > 0 ? end : 1;  // clamp target: slot lim - 1 is always valid
  lemoq_attn::issue_tokens<T>(ta, kb, vb, ksh, vsh, base, lim, tl, dl, D);
  lemoq_attn::SoftmaxState<T::EPL> st;
  lemoq_attn::softmax_init(st);
  while (base < end) {
    int64_t nb = base + STRIDE;
    lemoq_attn::issue_tokens<T>(tb, kb, vb, ksh, vsh, nb, lim, tl, dl, D);
    LEMOQ_LOADS_ISSUED();
    lemoq_attn::fold_tokens<T>(st, ta, qx, base, end, tl, lane, qk_scale);
    base = nb;
    if (base >= end) break;
    nb = base + STRIDE;
    lemoq_attn::issue_tokens<T>(ta, kb, vb, ksh, vsh, nb, lim, tl, dl, D);
    LEMOQ_LOADS_ISSUED();
    lemoq_attn::fold_tokens<T>(st, tb, qx, base, end, tl, lane, qk_scale);
    base = nb;
  }
  lemoq_attn::finish_split<T, NW, D>(st, wm, wl, wacc, lane, wave, tl, dl, (int64_t)h * NS + sp,
                                     m_out, l_out, acc_out);
}

// LSE merge of one head per block: the split weights 2^(m_j - M) and the
// denominator are formed once in LDS, then thread t streams acc[j][t] for all
// splits (independent loads, fixed split order).
__global__ __launch_bounds__(256) void attn_merge_kernel(const float* __restrict__ m,
                                                         const float* __restrict__ l,
                                                         const float* __restrict__ acc, int NS,
                                                         int D, uint16_t* __restrict__ out) {
  __shared__ float wj[1024];
  __shared__ float red[2];
  const int h = blockIdx.x;
  const float* mh = m + (int64_t)h * NS;
  const float* lh = l + (int64_t)h * NS;
  const float* ah = acc + (int64_t)h * NS * D;
  for (int j = threadIdx.x; j < NS; j += blockDim.x) wj[j] = mh[j];
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = -INFINITY;
    for (int j = 0; j < NS; ++j) M = fmaxf(M, wj[j]);
    if (!(M > -INFINITY)) M = 0.0f;  // every split empty: out = 0
    red[0] = M;
  }
  __syncthreads();
  const float M = red[0];
  for (int j = threadIdx.x; j < NS; j += blockDim.x) wj[j] = exp2f(wj[j] - M);
  __syncthreads();
  if (threadIdx.x == 0) {
    float den = 0.0f;
    for (int j = 0; j < NS; ++j) den += lh[j] * wj[j];
    red[1] = den;
  }
  __syncthreads();
  const float den = red[1];
  for (int t = threadIdx.x; t < D; t += blockDim.x) {
    float num = 0.0f;
    int j = 0;
    for (; j + 4 <= NS; j += 4) {
      const float a0 = ah[(int64_t)j * D + t], a1 = ah[(int64_t)(j + 1) * D + t];
      const float a2 = ah[(int64_t)(j + 2) * D + t], a3 = ah[(int64_t)(j + 3) * D + t];
      num += a0 * wj[j];
      num += a1 * wj[j + 1];
      num += a2 * wj[j + 2];
      num += a3 * wj[j + 3];
    }
    for (; j < NS; ++j) num += ah[(int64_t)j * D + t] * wj[j];
    out[(int64_t)h * D + t] = f2h(den > 0.0f ? num / den : num);
  }
}

// LSE merge with one wave per (head, 64 dims) and at most NSMAX splits: every
// load (lane j's m[j] and l[j], and acc[j][dims] of all splits) is issued at
// entry, so the merge waits on memory once; the wave forms M = max m_j,
// w_j = 2^(m_j - M) and den = sum l_j w_j with DPP reductions and broadcasts
// w_j with readlane.  No LDS, no barrier.  num = sum_j acc_j w_j in split
// order.  Slots j >= NS read a valid split (clamped) with weight 0.
template <int NSMAX>
__global__ __launch_bounds__(64) void attn_merge_wave_kernel(const float* __restrict__ m,
                                                             const float* __restrict__ l,
                                                             const float* __restrict__ acc,
                                                             int NS, int D,
                                                             uint16_t* __restrict__ out) {
  const int h = blockIdx.x, lane = threadIdx.x;
  const int t = blockIdx.y * 64 + lane;
  const int tc = t < D ? t : D - 1;
  const float* ah = acc + (int64_t)h * NS * D + tc;
  const int jl = lane < NS ? lane : NS - 1;
  const float mraw = m[(int64_t)h * NS + jl];
  const float lraw = l[(int64_t)h * NS + jl];
  float a[NSMAX];
#pragma unroll
  for (int j = 0; j < NSMAX; ++j) a[j] = ah[(int64_t)(j < NS ? j : NS - 1) * D];
  LEMOQ_LOADS_ISSUED();
  float den;
  const float wj = lemoq_attn::lse_weight(mraw, lraw, lane, NS, den);
  // Unconditional store: a lane with t >= D read the clamped column D - 1,
  // so it writes lane D-1's value to out[D-1] (identical bits).  A store
  // under `t < D` would let the compiler sink the acc loads and the sum into
  // the branch, after the reductions, costing a second memory round trip.
  out[(int64_t)h * D + tc] = lemoq_attn::lse_out<NSMAX>(a, wj, den);
}

template <bool I8>
int launch_split(hipStream_t st, const uint16_t* q, const void* k, const uint16_t* ks,
                 const void* v, const uint16_t* vs, int64_t head_stride, int64_t s_len,
                 int64_t max_len, const int32_t* filled, int64_t heads, int64_t D, int64_t NS,
                 float qk_scale, float* m, float* l, float* acc) {
  dim3 grid((unsigned)NS, (unsigned)heads);
#define LEMOQ_SPLIT_CASE(DD)                                                                   \
  case DD:                                                                                     \
    hipLaunchKernelGGL((attn_split_kernel<DD, I8>), grid, dim3(256), 0, st, q, k, ks, v, vs,  \
                       head_stride, s_len, max_len, filled, (int)NS, qk_scale, m, l, acc);    \
    break;
  switch (D) {
    LEMOQ_SPLIT_CASE(64)
    LEMOQ_SPLIT_CASE(128)
    LEMOQ_SPLIT_CASE(256)
    default: return LEMOQ_ERR_UNSUPPORTED;
  }
#undef LEMOQ_SPLIT_CASE
  LEMOQ_CHECK_LAUNCH();
}

int check_split_args(const void* q, const void* k, const void* v, const int32_t* filled,
                     const float* m, const float* l, const float* acc, int64_t heads, int64_t D,
                     int64_t NS, int64_t head_stride, int64_t max_len) {
  if (!q || !k || !v || !filled || !m || !l || !acc) return LEMOQ_ERR_NULL;
  if (heads <= 0 || heads > 65535 || NS <= 0 || NS > 65535) return LEMOQ_ERR_SHAPE;
  if (D != 64 && D != 128 && D != 256) return LEMOQ_ERR_UNSUPPORTED;
  if (max_len <= 0 || head_stride < max_len * D) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(q) || !lemoq_aligned16(k) || !lemoq_aligned16(v)) return LEMOQ_ERR_ALIGN;
  return LEMOQ_OK;
}

}  // namespace

// The f16 entry point has no separate capacity argument; the cache capacity
// is head_stride / D (the reference requires a non-overlapping head stride
// of at least S*D, src/lemoq/kernels/attn_decode.py:548-549).
extern "C" int lemoq_attn_split_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                    int64_t head_stride, const int32_t* filled, int64_t heads,
                                    int64_t head_dim, int64_t num_splits, float qk_scale,
                                    float* m, float* l, float* acc, void* stream) {
  if (head_dim <= 0) return LEMOQ_ERR_SHAPE;
  const int64_t max_len = head_stride / head_dim;
  int rc = check_split_args(q, k, v, filled, m, l, acc, heads, head_dim, num_splits, head_stride,
                            max_len);
  if (rc) return rc;
  if ((head_stride * 2) % 16 != 0) return LEMOQ_ERR_ALIGN;
  return launch_split<false>(lemoq_stream(stream), q, k, nullptr, v, nullptr, head_stride, 0,
                             max_len, filled, heads, head_dim, num_splits, qk_scale, m, l, acc);
}

extern "C" int lemoq_attn_split_i8(const uint16_t* q, const int8_t* kc, const uint16_t* ks,
                                   const int8_t* vc, const uint16_t* vs, int64_t head_stride,
                                   int64_t s_len, const int32_t* filled, int64_t heads,
                                   int64_t head_dim, int64_t num_splits, float qk_scale, float* m,
                                   float* l, float* acc, void* stream) {
  if (!ks || !vs) return LEMOQ_ERR_NULL;
  int rc = check_split_args(q, kc, vc, filled, m, l, acc, heads, head_dim, num_splits,
                            head_stride, s_len);
  if (rc) return rc;
  if (head_stride % 16 != 0) return LEMOQ_ERR_ALIGN;
  return launch_split<true>(lemoq_stream(stream), q, kc, ks, vc, vs, head_stride, s_len, s_len,
                            filled, heads, head_dim, num_splits, qk_scale, m, l, acc);
}

extern "C" int lemoq_attn_merge(const float* m, const float* l, const float* acc, int64_t heads,
                                int64_t num_splits, int64_t head_dim, uint16_t* out,
                                void* stream) {
  if (!m || !l || !acc || !out) return LEMOQ_ERR_NULL;
  if (heads <= 0 || heads > 65535 || num_splits <= 0 || num_splits > 1024 || head_dim <= 0 ||
      head_dim > 256)
    return LEMOQ_ERR_SHAPE;
  hipStream_t st = lemoq_stream(stream);
  if (num_splits <= 64) {
    const dim3 grid((unsigned)heads, (unsigned)((head_dim + 63) / 64));
    if (num_splits <= 16)
      hipLaunchKernelGGL((attn_merge_wave_kernel<16>), grid, dim3(64), 0, st, m, l, acc,
                         (int)num_splits, (int)head_dim, out);
    else
      hipLaunchKernelGGL((attn_merge_wave_kernel<64>), grid, dim3(64), 0, st, m, l, acc,
                         (int)num_splits, (int)head_dim, out);
    LEMOQ_CHECK_LAUNCH();
  }
  const int threads = head_dim <= 64 ? 64 : (head_dim <= 128 ? 128 : 256);
  hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)heads), dim3(threads), 0, st, m, l, acc,
                     (int)num_splits, (int)head_dim, out);
  LEMOQ_CHECK_LAUNCH();
}
