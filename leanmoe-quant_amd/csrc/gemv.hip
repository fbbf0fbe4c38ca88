// w8a16 dense GEMV (dequantisation in registers), the router (RMSNorm + fp16
// GEMV + softmax/top-k), routing top-k, and the greedy argmax that advances
// the decode position on the device.
//
// GEMV layout.  A 256-thread block is 4 independent waves; wave w of block b
// owns the R consecutive output rows (4b + w)*R ... and never synchronises
// with the other waves.  Each lane first issues every load it will need: the
// 16-byte code slices of its R rows (lane l reads bytes [1024j + 16l, +16) of
// chunk j of a row, fully coalesced) with their fp16 scales, then its slice
// of the activation row (and of the RMSNorm weight).  Only then does any
// arithmetic start: the RMSNorm of the prologue is a wave reduction over the
// slices (the wave holds the whole row), codes are turned into exact fp16
// pairs and reduced with v_dot2_f32_f16 in fp32, and a butterfly sums each
// row.  No LDS and no barrier stand between kernel entry and the weight
// stream.  No MFMA: at batch 1 this is ~1 flop per weight byte, HBM bound.
#include "common.h"

namespace {

struct GemvArgs {
  const uint16_t* x;
  int64_t x_ld;
  const int64_t* x_row_index;  // embedding gather: row *x_row_index of x
  int64_t x_rows;
  int K;
  const uint16_t* norm_w;  // RMSNorm prologue when non-null
  float eps;
  uint16_t* x_copy;  // block 0 / wave 0 stores the raw input row here
  const int8_t* codes;
  const uint16_t* scale;
  int64_t N;
  int Kp;
  int group;
  const uint16_t* resid;  // y = fp16(fp16(acc) + resid) when non-null
  void* y;
  int64_t y_ld;
  int y_f16;
  // argmax epilogue: per-block best (fp16-rounded value, lowest row)
  float* am_val;
  int32_t* am_idx;
};

constexpr int kArgmaxPlain = 0;
constexpr int kArgmaxPartials = 1;
constexpr int kArgmaxPartialsDq = 2;  // as kArgmaxPartials, weights rounded to fp16 before the dot

// Block epilogue of the argmax partials: each of the 4 waves brings its best
// (fp16-rounded value, lowest row; -inf / 0x7fffffff when it has no row) and
// thread 0 stores the block's best at blockIdx.x (ties -> lowest row; a block
// without a valid row stores -inf / -1).  Every thread of the block calls it.
__device__ __forceinline__ void block_argmax_partial(float bv, int bi, int wave, int lane, float* am_val,
                                                     int32_t* am_idx) {
  __shared__ float sv[4];
  __shared__ int si[4];
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    int i = si[0];
#pragma unroll
    for (int w = 1; w < 4; ++w)
      if (sv[w] > v || (sv[w] == v && si[w] < i)) {
        v = sv[w];
        i = si[w];
      }
    const bool none = i == 0x7fffffff;
    am_val[blockIdx.x] = none ? -INFINITY : v;
    am_idx[blockIdx.x] = none ? -1 : i;
  }
}

template <int KCH, int R, int MODE, bool EXACT>
__global__ __launch_bounds__(256) void gemv_w8_kernel(const GemvArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m = blockIdx.y;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * R;

  // Activation loads go first: the load counter retires in order, so the
  // prologue (RMSNorm) then waits only for them while the weights stream in.
  W8Tile<R, KCH> t;
  const uint16_t* xr;
  bool x_ok = true;
  if (a.x_row_index) {
    const int64_t r = a.x_row_index[0];
    x_ok = r >= 0 && r < a.x_rows;  // an index outside the table reads as a zero row
    xr = a.x + (x_ok ? r : 0) * a.x_ld;
  } else {
    xr = a.x + m * a.x_ld;
  }
  // The residual of this wave's rows is loaded now, not in the epilogue, so
  // the epilogue does not wait on memory (lane r < R holds row row0 + r).
  // The load is unconditional (a valid address when there is no residual):
  // a load under a branch is waited on right away, before the loads below
  // are issued.
  uint16_t res = 0;
  if (MODE == kArgmaxPlain) {
    const int64_t nr = row0 + (lane & (R - 1));
    const uint16_t* rp = a.resid ? a.resid + (nr < a.N ? nr : a.N - 1) : a.x;
    res = *rp;
  }
  XRaw<KCH> xv;
  // Exact shapes with K >= 2048: the RMSNorm prologue runs once per block
  // (8 values per thread, LDS), not once per wave, after the weight loads.
  constexpr bool kBlockNorm = EXACT && KCH >= 2;
  if (kBlockNorm && a.norm_w) {
    __shared__ __align__(16) uint16_t xs[KCH * 1024];
    __shared__ float red[4];
    constexpr int NV = KCH >= 2 ? KCH / 2 : 1;  // u32x4 (8 values) per thread
    u32x4 rv[NV], wv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int off = (i * 256 + threadIdx.x) * 8;
      rv[i] = *reinterpret_cast<const u32x4*>(xr + off);
      wv[i] = *reinterpret_cast<const u32x4*>(a.norm_w + off);
    }
    w8_issue<R, KCH, EXACT>(t, a.codes, a.scale, row0, a.N, a.Kp, a.Kp / a.group, a.group, lane);
    LEMOQ_LOADS_ISSUED();
    float ssq = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (!x_ok) rv[i] = (u32x4){0u, 0u, 0u, 0u};
      const uint32_t q[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float x0 = h2f((uint16_t)(q[k] & 0xFFFFu)), x1 = h2f((uint16_t)(q[k] >> 16));
        ssq = fmaf(x0, x0, ssq);
        ssq = fmaf(x1, x1, ssq);
      }
      if (a.x_copy && blockIdx.x == 0)
        *reinterpret_cast<u32x4*>(a.x_copy + (i * 256 + threadIdx.x) * 8) = rv[i];
    }
    ssq = wave_sum(ssq);
    if (lane == 0) red[wave] = ssq;
    __syncthreads();
    const float rstd = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)a.K + a.eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
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
    for (int j = 0; j < KCH; ++j) {
      xv.v[j][0] = *reinterpret_cast<const u32x4*>(xs + 1024 * j + 16 * lane);
      xv.v[j][1] = *reinterpret_cast<const u32x4*>(xs + 1024 * j + 16 * lane + 8);
    }
  } else {
    const bool vec = ((reinterpret_cast<uintptr_t>(xr) & 15u) == 0) && ((a.K & 7) == 0);
    x_issue<KCH, EXACT>(xv, xr, a.K, vec, lane);
    XRaw<KCH> nw;
    if (a.norm_w) {
      const bool nvec = ((reinterpret_cast<uintptr_t>(a.norm_w) & 15u) == 0) && ((a.K & 7) == 0);
      x_issue<KCH, EXACT>(nw, a.norm_w, a.K, nvec, lane);
    }
    w8_issue<R, KCH, EXACT>(t, a.codes, a.scale, row0, a.N, a.Kp, a.Kp / a.group, a.group, lane);
    LEMOQ_LOADS_ISSUED();
    if (!x_ok) {
#pragma unroll
      for (int j = 0; j < KCH; ++j) xv.v[j][0] = xv.v[j][1] = (u32x4){0u, 0u, 0u, 0u};
    }
    if (a.x_copy && blockIdx.x == 0 && wave == 0) {
#pragma unroll
      for (int j = 0; j < KCH; ++j) {
        const int off = 1024 * j + 16 * lane;
        const uint32_t w[8] = {xv.v[j][0].x, xv.v[j][0].y, xv.v[j][0].z, xv.v[j][0].w,
                               xv.v[j][1].x, xv.v[j][1].y, xv.v[j][1].z, xv.v[j][1].w};
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (off + i < a.K) a.x_copy[off + i] = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
      }
    }
    if (a.norm_w) x_rmsnorm<KCH>(xv, nw, a.K, a.eps);
  }
  XChunk xc[KCH];
  x_chunks<KCH>(xv, xc);

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    acc[r] = wave_sum(MODE == kArgmaxPartialsDq ? w8_row_dot_dq<R, KCH>(t, r, xc) : w8_row_dot<R, KCH>(t, r, xc));

  if (MODE == kArgmaxPlain) {
    if (lane < R) {
      float v = acc[0];
#pragma unroll
      for (int r = 1; r < R; ++r)
        if (lane == r) v = acc[r];
      const int64_t n = row0 + lane;
      if (n < a.N) {
        if (a.y_f16) {
          uint16_t o = f2h(v);
          if (a.resid) o = hadd_round(h2f(o), res);
          reinterpret_cast<uint16_t*>(a.y)[m * a.y_ld + n] = o;
        } else {
          reinterpret_cast<float*>(a.y)[m * a.y_ld + n] = v;
        }
      }
    }
  } else {
    // fp16 logits out, plus this block's best (value, lowest row).
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t n = row0 + r;
      const uint16_t o = f2h(acc[r]);
      if (n < a.N) {
        if (lane == r) reinterpret_cast<uint16_t*>(a.y)[n] = o;
        const float v = h2f(o);
        if (v > bv) {  // rows ascend: strict > keeps the lowest row on ties
          bv = v;
          bi = (int)n;
        }
      }
    }
    block_argmax_partial(bv, bi, wave, lane, a.am_val, a.am_idx);
  }
}

template <int KCH, int MODE>
int launch_gemv(int R, bool exact, dim3 grid, hipStream_t st, const GemvArgs& a) {
#define LEMOQ_GEMV_CASE(RR)                                                                     \
  case RR:                                                                                      \
    if (exact)                                                                                  \
      hipLaunchKernelGGL((gemv_w8_kernel<KCH, RR, MODE, true>), grid, dim3(256), 0, st, a);    \
    else                                                                                        \
      hipLaunchKernelGGL((gemv_w8_kernel<KCH, RR, MODE, false>), grid, dim3(256), 0, st, a);   \
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

// Rows per wave: 2 (swept on MI355X at the OLMoE shapes with cold weights:
// R = 1, 2, 4 for the 2048-, 6144- and 50304-row projections; 2 is best or
// within 2% everywhere).
int rows_per_wave(int64_t) { return 2; }

int kch_pow2(int64_t Kp) {
  const int64_t kch = (Kp + 1023) / 1024;
  return kch <= 1 ? 1 : (kch <= 2 ? 2 : (kch <= 4 ? 4 : 8));
}

template <int MODE>
int gemv_dispatch(hipStream_t st, GemvArgs a, int64_t M) {
  if (a.N <= 0 || M <= 0 || a.K <= 0) return LEMOQ_ERR_SHAPE;
  if (a.Kp > 8192 || a.Kp % 16 != 0 || a.group <= 0 || a.group % 16 != 0 || a.Kp % a.group != 0 ||
      a.K > a.Kp)
    return LEMOQ_ERR_UNSUPPORTED;
  if (M > 65535) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(a.codes)) return LEMOQ_ERR_ALIGN;
  const int R = rows_per_wave(a.N);
  const int64_t blocks = (a.N + 4 * R - 1) / (4 * R);
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  dim3 grid((unsigned)blocks, (unsigned)M);
  const int kch = kch_pow2(a.Kp);
  // Straight-line loads when the tile never leaves the matrix and the
  // activation rows are whole aligned 1 KB chunks.
  const bool exact = a.K == a.Kp && a.Kp == 1024 * kch && a.N % (4 * R) == 0 &&
                     lemoq_aligned16(a.x) && (M == 1 || a.x_ld % 8 == 0) &&
                     (a.x_row_index == nullptr || a.x_ld % 8 == 0) &&
                     (a.norm_w == nullptr || lemoq_aligned16(a.norm_w));
  switch (kch) {
    case 1: return launch_gemv<1, MODE>(R, exact, grid, st, a);
    case 2: return launch_gemv<2, MODE>(R, exact, grid, st, a);
    case 4: return launch_gemv<4, MODE>(R, exact, grid, st, a);
    default: return launch_gemv<8, MODE>(R, exact, grid, st, a);
  }
}

GemvArgs make_args(const uint16_t* x, int64_t x_ld, const int64_t* x_row_index, int64_t x_rows,
                   int64_t K, const uint16_t* norm_w, float eps, uint16_t* x_copy,
                   const int8_t* codes, const uint16_t* scale, int64_t N, int64_t Kp,
                   int64_t group, const uint16_t* resid, void* y, int64_t y_ld, int y_f16) {
  GemvArgs a;
  a.x = x;
  a.x_ld = x_ld;
  a.x_row_index = x_row_index;
  a.x_rows = x_rows;
  a.K = (int)K;
  a.norm_w = norm_w;
  a.eps = eps;
  a.x_copy = x_copy;
  a.codes = codes;
  a.scale = scale;
  a.N = N;
  a.Kp = (int)Kp;
  a.group = (int)group;
  a.resid = resid;
  a.y = y;
  a.y_ld = y_ld;
  a.y_f16 = y_f16;
  a.am_val = nullptr;
  a.am_idx = nullptr;
  return a;
}

// ---------------------------------------------------------------------------
// Greedy selection + step advance (one 1024-thread block) over either the
// fp16 logits themselves (PARTIALS == false: candidate i has value logits[i])
// or the per-block partials of the lm_head GEMV (value val[i], row idx[i]).
// Ties resolve to the lowest row; NaN never wins; all -inf/NaN -> row 0.
// Then: next = argmax, or prompt[*pos + 1] while *pos + 1 < prompt_len;
// *token = next, history[*pos + 1] = next, *pos += 1, *filled = *pos + 1.
// *pos and the prompt token it selects are loaded at entry, around the first
// pass of candidates, so the advance at the end waits on no memory; the wave
// reductions are DPP (largest value, then the lowest row among the lanes
// holding it).  n < 2^31.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ int wave_min_i32(int v) {
  v = min(v, dpp_i<LEMOQ_DPP_QUAD_1032>(v));
  v = min(v, dpp_i<LEMOQ_DPP_QUAD_2301>(v));
  v = min(v, dpp_i<LEMOQ_DPP_ROW_HALF_MIRROR>(v));
  v = min(v, dpp_i<LEMOQ_DPP_ROW_MIRROR>(v));
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

constexpr int kArgmaxPass = 8;  // candidate loads per thread per pass, all issued before comparing

template <bool PARTIALS>
__device__ __forceinline__ void argmax_load_pass(const uint16_t* __restrict__ logits,
                                                 const float* __restrict__ pv,
                                                 const int32_t* __restrict__ pi, int64_t n,
                                                 int64_t base, int tid, float (&v)[kArgmaxPass],
                                                 int (&ix)[kArgmaxPass]) {
#pragma unroll
  for (int j = 0; j < kArgmaxPass; ++j) {
    const int64_t i = base + (int64_t)j * 1024 + tid;
    const int64_t ic = i < n ? i : n - 1;  // clamped: every load is valid and unconditional
    v[j] = PARTIALS ? pv[ic] : h2f(logits[ic]);
    const int raw = PARTIALS ? pi[ic] : (int)ic;
    ix[j] = i < n ? raw : -1;
  }
}

__device__ __forceinline__ void argmax_fold_pass(const float (&v)[kArgmaxPass],
                                                 const int (&ix)[kArgmaxPass], float& bv, int& bi) {
#pragma unroll
  for (int j = 0; j < kArgmaxPass; ++j)
    if (ix[j] >= 0 && (v[j] > bv || (v[j] == bv && ix[j] < bi))) {
      bv = v[j];
      bi = ix[j];
    }
}

// fp16 logits with n % 8 == 0 and a 16-byte aligned row: 8 candidates per
// 16-byte load, kArgmaxPass loads per thread per pass (65536 candidates a pass,
// a 50304-row vocabulary in one).
__device__ __forceinline__ void argmax_load_pass_vec(const uint16_t* __restrict__ logits, int64_t nv,
                                                     int64_t vbase, int tid, u32x4 (&w)[kArgmaxPass]) {
#pragma unroll
  for (int j = 0; j < kArgmaxPass; ++j) {
    const int64_t q = vbase + (int64_t)j * 1024 + tid;
    w[j] = *reinterpret_cast<const u32x4*>(logits + (q < nv ? q : nv - 1) * 8);  // clamped, unconditional
  }
}

__device__ __forceinline__ void argmax_fold_pass_vec(const u32x4 (&w)[kArgmaxPass], int64_t nv, int64_t vbase,
                                                     int tid, float& bv, int& bi) {
#pragma unroll
  for (int j = 0; j < kArgmaxPass; ++j) {
    const int64_t q = vbase + (int64_t)j * 1024 + tid;
    if (q >= nv) continue;
    const uint32_t h[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float v = h2f((uint16_t)(h[k >> 1] >> (16 * (k & 1))));
      const int i = (int)(q * 8 + k);
      if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
      }
    }
  }
}

template <bool PARTIALS, bool VEC = false>
__global__ __launch_bounds__(1024) void argmax_advance_kernel(
    const uint16_t* __restrict__ logits, const float* __restrict__ pv,
    const int32_t* __restrict__ pi, int64_t n, int64_t* __restrict__ token,
    int64_t* __restrict__ pos, int32_t* __restrict__ filled, const int64_t* __restrict__ prompt,
    int64_t prompt_len, int64_t* __restrict__ history, int64_t history_len) {
  static_assert(!(PARTIALS && VEC), "the vector form reads fp16 logits");
  __shared__ float bvs[16];
  __shared__ int bis[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t p = pos[0];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  float v[kArgmaxPass];
  int ix[kArgmaxPass];
  u32x4 w[kArgmaxPass];
  const int64_t nv = n / 8;
  if constexpr (VEC)
    argmax_load_pass_vec(logits, nv, 0, tid, w);
  else
    argmax_load_pass<PARTIALS>(logits, pv, pi, n, 0, tid, v, ix);
  LEMOQ_LOADS_ISSUED();
  // The prompt token of position p + 1 (a valid address whether or not it is used).
  const bool feed = prompt && p + 1 >= 0 && p + 1 < prompt_len;
  const int64_t ptok = prompt ? prompt[feed ? p + 1 : 0] : 0;
  if constexpr (VEC) {
    argmax_fold_pass_vec(w, nv, 0, tid, bv, bi);
    for (int64_t vb = (int64_t)kArgmaxPass * 1024; vb < nv; vb += (int64_t)kArgmaxPass * 1024) {
      argmax_load_pass_vec(logits, nv, vb, tid, w);
      argmax_fold_pass_vec(w, nv, vb, tid, bv, bi);
    }
  } else {
    argmax_fold_pass(v, ix, bv, bi);
    for (int64_t base = (int64_t)kArgmaxPass * 1024; base < n; base += (int64_t)kArgmaxPass * 1024) {
      argmax_load_pass<PARTIALS>(logits, pv, pi, n, base, tid, v, ix);
      argmax_fold_pass(v, ix, bv, bi);
    }
  }
  // NaN is never held (every comparison with it is false), so the wave max is
  // a real value or -inf; lanes holding it offer their lowest row.
  const float M = wave_max(bv);
  const int I = wave_min_i32(bv == M ? bi : 0x7fffffff);
  if (lane == 0) {
    bvs[wave] = M;
    bis[wave] = I;
  }
  __syncthreads();
  if (tid == 0) {
    float bm = bvs[0];
    int idx = bis[0];
    for (int w = 1; w < 16; ++w) {
      if (bvs[w] > bm || (bvs[w] == bm && bis[w] < idx)) {
        bm = bvs[w];
        idx = bis[w];
      }
    }
    if (idx == 0x7fffffff || idx < 0) idx = 0;  // every logit was -inf or NaN
    const int64_t next = feed ? ptok : (int64_t)idx;
    token[0] = next;
    if (history && p + 1 >= 0 && p + 1 < history_len) history[p + 1] = next;
    pos[0] = p + 1;
    filled[0] = (int32_t)(p + 2);
  }
}

// ---------------------------------------------------------------------------
// Router of one token in one 1024-thread block: xn = RMSNorm(h) and
// logits[e] = fp16(xn . W[e]) with fp32 accumulation (the F.linear of
// moe_static._route, src/lemoq/kernels/moe_static.py:262-283, on the
// post-attention norm's output), then wave 0 routes (softmax, top_k, optional
// renorm) and writes ids and weights.  Wave w streams rows w*4 .. w*4+3 of
// each 64-row pass, issuing all of its loads (rows, h, norm weight) first; it
// recomputes the norm from its own slices (the wave holds the whole row).
// ---------------------------------------------------------------------------
template <int KCH, bool EXACT>
__global__ __launch_bounds__(1024) void router_kernel(
    const uint16_t* __restrict__ h, const uint16_t* __restrict__ norm_w, float eps, int H,
    const uint16_t* __restrict__ rw, int E, int top_k, int norm, uint16_t* __restrict__ xn_out,
    uint16_t* __restrict__ logits_out, float* __restrict__ top_w32,
    uint16_t* __restrict__ top_w16, int64_t* __restrict__ top_i) {
  __shared__ float lg[1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  XRaw<KCH> xv, nw;
  bool normed = false;
  for (int e0 = wave * 4; e0 < E; e0 += 64) {
    XRaw<KCH> wr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = e0 + r < E ? e0 + r : E - 1;
      x_issue<KCH, EXACT>(wr[r], rw + (int64_t)e * H, H, true, lane);
    }
    if (!normed) {
      x_issue<KCH, EXACT>(xv, h, H, true, lane);
      if (norm_w) x_issue<KCH, EXACT>(nw, norm_w, H, true, lane);
    }
    LEMOQ_LOADS_ISSUED();
    if (!normed) {
      if (norm_w) x_rmsnorm<KCH>(xv, nw, H, eps);
      normed = true;
      if (xn_out && wave == 0) {
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
          const int off = 1024 * j + 16 * lane;
          if (off + 16 <= H) {
            *reinterpret_cast<u32x4*>(xn_out + off) = xv.v[j][0];
            *reinterpret_cast<u32x4*>(xn_out + off + 8) = xv.v[j][1];
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < KCH; ++j)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const uint32_t ww[4] = {wr[r].v[j][q].x, wr[r].v[j][q].y, wr[r].v[j][q].z, wr[r].v[j][q].w};
          const uint32_t xw[4] = {xv.v[j][q].x, xv.v[j][q].y, xv.v[j][q].z, xv.v[j][q].w};
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc = __builtin_amdgcn_fdot2(as_h2(ww[i]), as_h2(xw[i]), acc, false);
        }
      acc = wave_sum(acc);
      const int e = e0 + r;
      if (lane == 0 && e < E) {
        const uint16_t o = f2h(acc);
        lg[e] = h2f(o);
        if (logits_out) logits_out[e] = o;
      }
    }
  }
  __syncthreads();
  if (wave == 0) {
    int id;
    float w;
    if (E <= 64) {
      float z[1] = {lane < E ? lg[lane] : -INFINITY};
      wave_route<1>(z, E, top_k, norm != 0, id, w);
    } else {
      float z[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) z[i] = lane + 64 * i < E ? lg[lane + 64 * i] : -INFINITY;
      wave_route<16>(z, E, top_k, norm != 0, id, w);
    }
    if (lane < top_k) {
      top_i[lane] = (int64_t)id;
      if (top_w32) top_w32[lane] = w;
      if (top_w16) top_w16[lane] = f2h(w);
    }
  }
}

// ---------------------------------------------------------------------------
// Router logits of one token over many blocks: one wave per expert row; every
// wave recomputes xn = RMSNorm(h) from its own slices (the wave holds the
// whole row), so waves never synchronise.  logits[e] = fp16(xn . W[e]) with
// fp32 accumulation.  Wave 0 of block 0 stores xn.
// ---------------------------------------------------------------------------
template <int KCH, bool EXACT>
__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ h, const uint16_t* __restrict__ norm_w, float eps, int H,
    const uint16_t* __restrict__ rw, int E, uint16_t* __restrict__ xn_out,
    uint16_t* __restrict__ logits_out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x * 4 + wave;
  const int ec = e < E ? e : E - 1;
  XRaw<KCH> wr, xv, nw;
  x_issue<KCH, EXACT>(xv, h, H, true, lane);
  if (norm_w) x_issue<KCH, EXACT>(nw, norm_w, H, true, lane);
  x_issue<KCH, EXACT>(wr, rw + (int64_t)ec * H, H, true, lane);
  LEMOQ_LOADS_ISSUED();
  if (norm_w) x_rmsnorm<KCH>(xv, nw, H, eps);
  if (xn_out && blockIdx.x == 0 && wave == 0) {
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int off = 1024 * j + 16 * lane;
      if (off + 16 <= H) {
        *reinterpret_cast<u32x4*>(xn_out + off) = xv.v[j][0];
        *reinterpret_cast<u32x4*>(xn_out + off + 8) = xv.v[j][1];
      }
    }
  }
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < KCH; ++j)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t ww[4] = {wr.v[j][q].x, wr.v[j][q].y, wr.v[j][q].z, wr.v[j][q].w};
      const uint32_t xw[4] = {xv.v[j][q].x, xv.v[j][q].y, xv.v[j][q].z, xv.v[j][q].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2(as_h2(ww[i]), as_h2(xw[i]), acc, false);
    }
  acc = wave_sum(acc);
  if (lane == 0 && e < E) logits_out[e] = f2h(acc);
}

// fp16 lm_head of one token with the argmax partials: wave w of block b owns
// the 2 rows (4b + w)*2, +1, normalises x once for both (the router's
// x_rmsnorm), and each row's logit is fp16(xn . W[n]) with the router
// kernel's lane order and butterfly, so the logits equal
// router_logits_kernel's bit for bit.  Each block stores its best (value,
// lowest row) for argmax_advance_kernel<true>; the row count per block is
// the W8 lm_head's, so lemoq_lm_head_argmax_parts(N) sizes both.
template <int KCH, bool EXACT>
__global__ __launch_bounds__(256) void lm_head_f16_argmax_kernel(
    const uint16_t* __restrict__ h, const uint16_t* __restrict__ norm_w, float eps, int H,
    const uint16_t* __restrict__ w, int64_t N, uint16_t* __restrict__ logits, float* __restrict__ am_val,
    int32_t* __restrict__ am_idx) {
  constexpr int R = 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * R;
  XRaw<KCH> xv, nw, wr[R];
  x_issue<KCH, EXACT>(xv, h, H, true, lane);
  if (norm_w) x_issue<KCH, EXACT>(nw, norm_w, H, true, lane);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t n = row0 + r < N ? row0 + r : N - 1;
    x_issue<KCH, EXACT>(wr[r], w + n * H, H, true, lane);
  }
  LEMOQ_LOADS_ISSUED();
  if (norm_w) x_rmsnorm<KCH>(xv, nw, H, eps);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < KCH; ++j)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t ww[4] = {wr[r].v[j][q].x, wr[r].v[j][q].y, wr[r].v[j][q].z, wr[r].v[j][q].w};
        const uint32_t xw[4] = {xv.v[j][q].x, xv.v[j][q].y, xv.v[j][q].z, xv.v[j][q].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2(as_h2(ww[i]), as_h2(xw[i]), acc, false);
      }
    const uint16_t o = f2h(wave_sum(acc));
    const int64_t n = row0 + r;
    if (n < N) {
      if (lane == r) logits[n] = o;
      const float v = h2f(o);
      if (v > bv) {  // rows ascend: strict > keeps the lowest row on ties
        bv = v;
        bi = (int)n;
      }
    }
  }
  block_argmax_partial(bv, bi, wave, lane, am_val, am_idx);
}

int launch_router_logits(hipStream_t st, const uint16_t* h, const uint16_t* norm_w, float eps,
                         int64_t H, const uint16_t* rw, int64_t E, uint16_t* xn_out,
                         uint16_t* logits) {
  const dim3 grid((unsigned)((E + 3) / 4));
  const int kch = kch_pow2(H);
  const bool exact = H == 1024 * kch;
#define LEMOQ_RL_CASE(KK)                                                                        \
  case KK:                                                                                       \
    if (exact)                                                                                   \
      hipLaunchKernelGGL((router_logits_kernel<KK, true>), grid, dim3(256), 0, st, h, norm_w,    \
                         eps, (int)H, rw, (int)E, xn_out, logits);                               \
    else                                                                                         \
      hipLaunchKernelGGL((router_logits_kernel<KK, false>), grid, dim3(256), 0, st, h, norm_w,   \
                         eps, (int)H, rw, (int)E, xn_out, logits);                               \
    break;
  switch (kch) {
    LEMOQ_RL_CASE(1)
    LEMOQ_RL_CASE(2)
    LEMOQ_RL_CASE(4)
    LEMOQ_RL_CASE(8)
    default: return LEMOQ_ERR_UNSUPPORTED;
  }
#undef LEMOQ_RL_CASE
  LEMOQ_CHECK_LAUNCH();
}

// Routing of T tokens, one wave per token (values per lane PL = ceil(E/64)).
// Logit kinds: fp32, fp16, or `splits` fp32 split-K partial planes of T x
// stride (the logit is fp16(sum of the planes in order, from 0), the finish
// of lemoq_gemm_f16_splitk, so routing the partials equals routing its output).
constexpr int kLogitsF32 = 0, kLogitsF16 = 1, kLogitsSplitK = 2;

template <int PL>
__global__ __launch_bounds__(256) void route_topk_kernel(const void* __restrict__ logits, int kind,
                                                         int64_t T, int E, int64_t stride, int splits,
                                                         int top_k, int norm,
                                                         float* __restrict__ top_w32,
                                                         uint16_t* __restrict__ top_w16,
                                                         int64_t* __restrict__ top_i) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int lane = threadIdx.x & 63;
  float z[PL];
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int idx = lane + 64 * i;
    if (idx < E) {
      if (kind == kLogitsSplitK) {
        // The planes' loads are all issued before the first add (a load per
        // loop trip would make each plane one more dependent memory round
        // trip); the sum stays in plane order from 0.
        const float* pp = reinterpret_cast<const float*>(logits) + t * stride + idx;
        constexpr int NP = 8;
        float pv[NP];
#pragma unroll
        for (int zz = 0; zz < NP; ++zz) pv[zz] = zz < splits ? pp[(int64_t)zz * T * stride] : 0.0f;
        float v = 0.0f;
#pragma unroll
        for (int zz = 0; zz < NP; ++zz)
          if (zz < splits) v += pv[zz];
        for (int zz = NP; zz < splits; ++zz) v += pp[(int64_t)zz * T * stride];
        z[i] = h2f(f2h(v));
      } else {
        z[i] = kind == kLogitsF16 ? h2f(reinterpret_cast<const uint16_t*>(logits)[t * stride + idx])
                                  : reinterpret_cast<const float*>(logits)[t * stride + idx];
      }
    } else {
      z[i] = -INFINITY;
    }
  }
  int id;
  float w;
  wave_route<PL>(z, E, top_k, norm != 0, id, w);
  if (lane < top_k) {
    top_i[t * top_k + lane] = (int64_t)id;
    if (top_w32) top_w32[t * top_k + lane] = w;
    if (top_w16) top_w16[t * top_k + lane] = f2h(w);
  }
}

int launch_route(hipStream_t st, const void* logits, int kind, int64_t T, int64_t E,
                 int64_t stride, int64_t top_k, int norm, float* w32, uint16_t* w16,
                 int64_t* ids, int splits = 1) {
  const int64_t blocks = (T + 3) / 4;
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  const int pl = (int)((E + 63) / 64);
#define LEMOQ_ROUTE_CASE(PP)                                                                    \
  if (pl <= PP) {                                                                               \
    hipLaunchKernelGGL((route_topk_kernel<PP>), dim3((unsigned)blocks), dim3(256), 0, st,      \
                       logits, kind, T, (int)E, stride, splits, (int)top_k, norm, w32, w16, ids); \
    LEMOQ_CHECK_LAUNCH();                                                                       \
  }
  LEMOQ_ROUTE_CASE(1)
  LEMOQ_ROUTE_CASE(4)
  LEMOQ_ROUTE_CASE(16)
#undef LEMOQ_ROUTE_CASE
  return LEMOQ_ERR_UNSUPPORTED;
}

int launch_router(hipStream_t st, const uint16_t* h, const uint16_t* norm_w, float eps, int64_t H,
                  const uint16_t* rw, int64_t E, int64_t top_k, int norm, uint16_t* xn_out,
                  uint16_t* logits, float* w32, uint16_t* w16, int64_t* ids) {
  const int kch = kch_pow2(H);
  const bool exact = H == 1024 * kch;
#define LEMOQ_ROUTER_CASE(KK)                                                                    \
  case KK:                                                                                       \
    if (exact)                                                                                   \
      hipLaunchKernelGGL((router_kernel<KK, true>), dim3(1), dim3(1024), 0, st, h, norm_w, eps,  \
                         (int)H, rw, (int)E, (int)top_k, norm, xn_out, logits, w32, w16, ids);   \
    else                                                                                         \
      hipLaunchKernelGGL((router_kernel<KK, false>), dim3(1), dim3(1024), 0, st, h, norm_w, eps, \
                         (int)H, rw, (int)E, (int)top_k, norm, xn_out, logits, w32, w16, ids);   \
    break;
  switch (kch) {
    LEMOQ_ROUTER_CASE(1)
    LEMOQ_ROUTER_CASE(2)
    LEMOQ_ROUTER_CASE(4)
    LEMOQ_ROUTER_CASE(8)
    default: return LEMOQ_ERR_UNSUPPORTED;
  }
#undef LEMOQ_ROUTER_CASE
  LEMOQ_CHECK_LAUNCH();
}

}  // namespace

extern "C" int lemoq_gemv_w8(const uint16_t* x, int64_t M, int64_t K, const int8_t* codes,
                             const uint16_t* scale, int64_t N, int64_t padded_k, int64_t group,
                             void* y, int y_is_f16, void* stream) {
  if (!x || !codes || !scale || !y) return LEMOQ_ERR_NULL;
  return gemv_dispatch<kArgmaxPlain>(
      lemoq_stream(stream),
      make_args(x, K, nullptr, 0, K, nullptr, 0.0f, nullptr, codes, scale, N, padded_k, group,
                nullptr, y, N, y_is_f16 ? 1 : 0),
      M);
}

extern "C" int lemoq_gemv_w8_fused(const uint16_t* x_src, const int64_t* x_row_index,
                                   int64_t x_rows, const uint16_t* norm_w, float eps,
                                   uint16_t* x_copy, const int8_t* codes, const uint16_t* scale,
                                   int64_t N, int64_t K, int64_t group, const uint16_t* residual,
                                   uint16_t* y, void* stream) {
  if (!x_src || !codes || !scale || !y) return LEMOQ_ERR_NULL;
  if (x_row_index && x_rows <= 0) return LEMOQ_ERR_SHAPE;
  return gemv_dispatch<kArgmaxPlain>(
      lemoq_stream(stream),
      make_args(x_src, K, x_row_index, x_rows, K, norm_w, eps, x_copy, codes, scale, N, K, group,
                residual, y, N, 1),
      1);
}

namespace {
template <int MODE>
int lm_head_argmax(const uint16_t* x, const uint16_t* norm_w, float eps, const int8_t* codes,
                   const uint16_t* scale, int64_t N, int64_t K, int64_t group, uint16_t* logits,
                   float* part_val, int32_t* part_idx, int64_t part_len, int64_t* token, int64_t* pos,
                   int32_t* filled, const int64_t* prompt, int64_t prompt_len, int64_t* history,
                   int64_t history_len, void* stream) {
  if (!x || !codes || !scale || !logits || !part_val || !part_idx || !token || !pos || !filled)
    return LEMOQ_ERR_NULL;
  if (N <= 0 || N > 0x7ffffffeLL) return LEMOQ_ERR_SHAPE;
  const int64_t blocks = (N + 4 * rows_per_wave(N) - 1) / (4 * rows_per_wave(N));
  if (part_len < blocks) return LEMOQ_ERR_SHAPE;
  GemvArgs a = make_args(x, K, nullptr, 0, K, norm_w, eps, nullptr, codes, scale, N, K, group,
                         nullptr, logits, N, 1);
  a.am_val = part_val;
  a.am_idx = part_idx;
  hipStream_t st = lemoq_stream(stream);
  const int rc = gemv_dispatch<MODE>(st, a, 1);
  if (rc) return rc;
  hipLaunchKernelGGL((argmax_advance_kernel<true>), dim3(1), dim3(1024), 0, st, nullptr, part_val,
                     part_idx, blocks, token, pos, filled, prompt, prompt_len, history,
                     history_len);
  LEMOQ_CHECK_LAUNCH();
}
}  // namespace

extern "C" int lemoq_lm_head_argmax_w8(const uint16_t* x, const uint16_t* norm_w, float eps,
                                       const int8_t* codes, const uint16_t* scale, int64_t N,
                                       int64_t K, int64_t group, uint16_t* logits,
                                       float* part_val, int32_t* part_idx, int64_t part_len,
                                       int64_t* token, int64_t* pos, int32_t* filled,
                                       const int64_t* prompt, int64_t prompt_len,
                                       int64_t* history, int64_t history_len, void* stream) {
  return lm_head_argmax<kArgmaxPartials>(x, norm_w, eps, codes, scale, N, K, group, logits, part_val,
                                         part_idx, part_len, token, pos, filled, prompt, prompt_len,
                                         history, history_len, stream);
}

extern "C" int lemoq_lm_head_argmax_w8_dq(const uint16_t* x, const uint16_t* norm_w, float eps,
                                          const int8_t* codes, const uint16_t* scale, int64_t N,
                                          int64_t K, int64_t group, uint16_t* logits,
                                          float* part_val, int32_t* part_idx, int64_t part_len,
                                          int64_t* token, int64_t* pos, int32_t* filled,
                                          const int64_t* prompt, int64_t prompt_len,
                                          int64_t* history, int64_t history_len, void* stream) {
  return lm_head_argmax<kArgmaxPartialsDq>(x, norm_w, eps, codes, scale, N, K, group, logits, part_val,
                                           part_idx, part_len, token, pos, filled, prompt, prompt_len,
                                           history, history_len, stream);
}

extern "C" int lemoq_lm_head_argmax_f16(const uint16_t* x, const uint16_t* norm_w, float eps,
                                        const uint16_t* weight, int64_t N, int64_t K, uint16_t* logits,
                                        float* part_val, int32_t* part_idx, int64_t part_len,
                                        int64_t* token, int64_t* pos, int32_t* filled,
                                        const int64_t* prompt, int64_t prompt_len, int64_t* history,
                                        int64_t history_len, void* stream) {
  if (!x || !weight || !logits || !part_val || !part_idx || !token || !pos || !filled)
    return LEMOQ_ERR_NULL;
  if (K <= 0 || K > 8192 || K % 16 != 0) return LEMOQ_ERR_UNSUPPORTED;
  if (N <= 0 || N > 0x7ffffffeLL) return LEMOQ_ERR_SHAPE;
  const int64_t blocks = lemoq_lm_head_argmax_parts(N);
  if (part_len < blocks) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(x) || !lemoq_aligned16(weight) || (norm_w && !lemoq_aligned16(norm_w)))
    return LEMOQ_ERR_ALIGN;
  hipStream_t st = lemoq_stream(stream);
  const int kch = kch_pow2(K);
  const bool exact = K == 1024 * kch;
#define LEMOQ_LMF_CASE(KK)                                                                          \
  case KK:                                                                                          \
    if (exact)                                                                                      \
      hipLaunchKernelGGL((lm_head_f16_argmax_kernel<KK, true>), dim3((unsigned)blocks), dim3(256), 0, st, x, \
                         norm_w, eps, (int)K, weight, N, logits, part_val, part_idx);                \
    else                                                                                            \
      hipLaunchKernelGGL((lm_head_f16_argmax_kernel<KK, false>), dim3((unsigned)blocks), dim3(256), 0, st, x, \
                         norm_w, eps, (int)K, weight, N, logits, part_val, part_idx);                \
    break;
  switch (kch) {
    LEMOQ_LMF_CASE(1)
    LEMOQ_LMF_CASE(2)
    LEMOQ_LMF_CASE(4)
    LEMOQ_LMF_CASE(8)
    default: return LEMOQ_ERR_UNSUPPORTED;
  }
#undef LEMOQ_LMF_CASE
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL((argmax_advance_kernel<true>), dim3(1), dim3(1024), 0, st, nullptr, part_val, part_idx,
                     blocks, token, pos, filled, prompt, prompt_len, history, history_len);
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int64_t lemoq_lm_head_argmax_parts(int64_t N) {
  if (N <= 0) return 0;
  return (N + 4 * rows_per_wave(N) - 1) / (4 * rows_per_wave(N));
}

extern "C" int lemoq_route_topk(const void* logits, int logits_is_f16, int64_t T, int64_t E,
                                int64_t row_stride, int64_t top_k, int norm_topk_prob,
                                float* top_w, int64_t* top_i, void* stream) {
  if (!logits || !top_w || !top_i) return LEMOQ_ERR_NULL;
  if (T < 0 || E <= 0 || E > 1024 || top_k <= 0 || top_k > E || top_k > 64 || row_stride < E)
    return LEMOQ_ERR_SHAPE;
  if (T == 0) return LEMOQ_OK;
  return launch_route(lemoq_stream(stream), logits, logits_is_f16 ? kLogitsF16 : kLogitsF32, T, E, row_stride,
                      top_k, norm_topk_prob ? 1 : 0, top_w, nullptr, top_i);
}

extern "C" int lemoq_route_topk_splitk(const float* partials, int64_t splits, int64_t T, int64_t E,
                                       int64_t top_k, int norm_topk_prob, float* top_w, int64_t* top_i,
                                       void* stream) {
  if (!partials || !top_w || !top_i) return LEMOQ_ERR_NULL;
  if (T < 0 || E <= 0 || E > 1024 || top_k <= 0 || top_k > E || top_k > 64 || splits < 1 || splits > 64)
    return LEMOQ_ERR_SHAPE;
  if (T == 0) return LEMOQ_OK;
  return launch_route(lemoq_stream(stream), partials, kLogitsSplitK, T, E, E, top_k, norm_topk_prob ? 1 : 0,
                      top_w, nullptr, top_i, (int)splits);
}

extern "C" int lemoq_router_logits(const uint16_t* h, const uint16_t* norm_w, float eps,
                                   int64_t hidden, const uint16_t* router_w, int64_t E,
                                   uint16_t* xn_out, uint16_t* logits_out, void* stream) {
  if (!h || !router_w || !logits_out) return LEMOQ_ERR_NULL;
  if (hidden <= 0 || hidden > 8192 || hidden % 16 != 0) return LEMOQ_ERR_UNSUPPORTED;
  if (E <= 0 || E > 65536) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(router_w) || !lemoq_aligned16(h) || (norm_w && !lemoq_aligned16(norm_w)) ||
      (xn_out && !lemoq_aligned16(xn_out)))
    return LEMOQ_ERR_ALIGN;
  return launch_router_logits(lemoq_stream(stream), h, norm_w, eps, hidden, router_w, E, xn_out,
                              logits_out);
}

extern "C" int lemoq_router_topk_fused(const uint16_t* h, const uint16_t* norm_w, float eps,
                                       int64_t hidden, const uint16_t* router_w, int64_t E,
                                       int64_t top_k, int norm_topk_prob, uint16_t* xn_out,
                                       uint16_t* logits_out, float* top_w_f32,
                                       uint16_t* top_w_f16, int64_t* top_i, void* stream) {
  if (!h || !router_w || !top_i) return LEMOQ_ERR_NULL;
  if (hidden <= 0 || hidden > 8192 || hidden % 16 != 0) return LEMOQ_ERR_UNSUPPORTED;
  if (E <= 0 || E > 1024 || top_k <= 0 || top_k > E || top_k > 64) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(router_w) || !lemoq_aligned16(h) || (norm_w && !lemoq_aligned16(norm_w)) ||
      (xn_out && !lemoq_aligned16(xn_out)))
    return LEMOQ_ERR_ALIGN;
  return launch_router(lemoq_stream(stream), h, norm_w, eps, hidden, router_w, E, top_k,
                       norm_topk_prob ? 1 : 0, xn_out, logits_out, top_w_f32, top_w_f16, top_i);
}

extern "C" int lemoq_argmax_advance(const uint16_t* logits, int64_t n, int64_t* token,
                                    int64_t* pos, int32_t* filled, const int64_t* prompt,
                                    int64_t prompt_len, int64_t* history, int64_t history_len,
                                    void* stream) {
  if (!logits || !token || !pos || !filled) return LEMOQ_ERR_NULL;
  if (n <= 0 || n > 0x7ffffffeLL) return LEMOQ_ERR_SHAPE;
  if (n % 8 == 0 && lemoq_aligned16(logits))
    hipLaunchKernelGGL((argmax_advance_kernel<false, true>), dim3(1), dim3(1024), 0, lemoq_stream(stream),
                       logits, nullptr, nullptr, n, token, pos, filled, prompt, prompt_len, history,
                       history_len);
  else
    hipLaunchKernelGGL((argmax_advance_kernel<false, false>), dim3(1), dim3(1024), 0, lemoq_stream(stream),
                       logits, nullptr, nullptr, n, token, pos, filled, prompt, prompt_len, history,
                       history_len);
  LEMOQ_CHECK_LAUNCH();
}
