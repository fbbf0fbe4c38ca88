// RMSNorm, RoPE, and the fused per-layer attention prologue of the decode
// step (q_norm/k_norm -> RoPE -> KV-INT8 write).
//
// RMSNorm rounding points follow HF OlmoeRMSNorm.forward as restated by the
// reference kernel (src/lemoq/kernels/rmsnorm.py:184-202): fp32 mean of
// squares, x*rstd rounded to fp16, then the fp16 product with the fp16 weight
// (exact in fp32, rounded once).  RoPE follows _rope_one_kernel
// (src/lemoq/kernels/rope.py:101-123): y = x*cos + sign*x[shift]*sin in fp32
// with rotate_half's halves, rounded to fp16.
#include "common.h"

namespace {

// VEC: rows held as 16-byte chunks in registers (H % 8 == 0, H <= 8192,
// x, w, y 16-byte aligned): one read of the row, 16-byte stores.
template <bool VEC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x, int H,
                                                      const uint16_t* __restrict__ w, float eps,
                                                      uint16_t* __restrict__ y) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  if constexpr (VEC) {
    u32x4 xv[RN_CHUNKS];
    rmsnorm_load_chunks(x + r * H, H, xv);
    rmsnorm_chunks(xv, H, w, eps, y + r * H, red);
  } else {
    rmsnorm_row_256(x + r * H, H, w, eps, y + r * H, red);
  }
}

// Embedding rows of several tokens: dst[r] = src[ids[r]] (a zero row for an
// id outside [0, n_rows)), 16 bytes per thread.
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint16_t* __restrict__ src,
                                                          int64_t n_rows, int64_t H,
                                                          const int64_t* __restrict__ ids,
                                                          uint16_t* __restrict__ dst) {
  const int64_t r = blockIdx.x;
  const int64_t id = ids[r];
  const bool ok = id >= 0 && id < n_rows;
  const uint16_t* s = src + (ok ? id : 0) * H;
  for (int64_t c = (int64_t)threadIdx.x * 8; c < H; c += 256 * 8) {
    u32x4 v = *reinterpret_cast<const u32x4*>(s + c);
    if (!ok) v = (u32x4){0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(dst + r * H + c) = v;
  }
}

__device__ __forceinline__ float rope_elem(float x, float xs, float c, float s, bool first_half) {
  return first_half ? x * c + (-xs) * s : x * c + xs * s;
}

__global__ __launch_bounds__(128) void rope_kernel(const uint16_t* __restrict__ x, int64_t x_sh,
                                                   int64_t x_sd, int D,
                                                   const uint16_t* __restrict__ cs,
                                                   const uint16_t* __restrict__ sn, int64_t cs_sd,
                                                   uint16_t* __restrict__ out, int64_t o_sh,
                                                   int64_t o_sd) {
  const int h = blockIdx.x;
  const int half = D / 2;
  for (int d = threadIdx.x; d < D; d += 128) {
    const bool first = d < half;
    const int sh = first ? d + half : d - half;
    const float xv = h2f(x[h * x_sh + d * x_sd]);
    const float xs = h2f(x[h * x_sh + sh * x_sd]);
    const float c = h2f(cs[d * cs_sd]);
    const float s = h2f(sn[d * cs_sd]);
    out[h * o_sh + d * o_sd] = f2h(rope_elem(xv, xs, c, s, first));
  }
}

// Fused attention prologue, one wave per (row kind, head): blocks
// [0, heads) take the q heads, [heads, 2*heads) the k heads, [2*heads,
// 3*heads) the v heads.  A q/k wave reads the whole heads*D row (the RMSNorm
// is over all heads, as HF's q_norm/k_norm over hidden_size) to form the sum
// of squares, then normalises and rotates only its own head: lane l holds
// elements d = l*EPL + i (EPL = D/64) and the rotate_half partner d +- D/2
// sits in lane l ^ 32.  k and v heads are quantised to KV-INT8 at slot *pos
// (amax / 127 scale, round-half-even codes; the arithmetic of
// src/lemoq/kernels/kv_int8.py:196-216).
template <int EPL>
__global__ __launch_bounds__(64) void qk_norm_rope_kv_kernel(
    const uint16_t* __restrict__ qkv, int heads, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, float eps, const uint16_t* __restrict__ cos_tab,
    const uint16_t* __restrict__ sin_tab, const int64_t* __restrict__ pos_ptr,
    uint16_t* __restrict__ q_out, int8_t* __restrict__ kc, uint16_t* __restrict__ ks,
    int8_t* __restrict__ vc, uint16_t* __restrict__ vs, int64_t code_head_stride, int64_t s_len,
    uint16_t* __restrict__ k_f16, uint16_t* __restrict__ v_f16, int64_t f16_head_stride,
    uint16_t* __restrict__ k_rot_out, float clip) {
  constexpr int D = 64 * EPL;
  const float clip16 = h2f(f2h(clip));
  const int lane = threadIdx.x;
  const int which = blockIdx.x / heads;  // 0 q, 1 k, 2 v
  const int h = blockIdx.x - which * heads;
  const int HD = heads * D;
  const int64_t pos = pos_ptr[0];
  const bool pos_ok = pos >= 0 && pos < s_len;
  const uint16_t* src = qkv + (int64_t)which * HD;
  const int d0 = lane * EPL;

  // own head's elements, raw
  float xv[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) xv[i] = h2f(src[h * D + d0 + i]);

  float o[EPL];
  if (which < 2) {
    const uint16_t* nw = which == 0 ? qn_w : kn_w;
    float wv[EPL], cv[EPL], sv[EPL];
    const int64_t prow = pos_ok ? pos : 0;  // clamped table read; writes need pos_ok
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      wv[i] = h2f(nw[h * D + d0 + i]);
      cv[i] = h2f(cos_tab[prow * D + d0 + i]);
      sv[i] = h2f(sin_tab[prow * D + d0 + i]);
    }
    // Slices lane*8 + 512 j in order, four v_dot2 each (ssq_f16x8): the
    // order the fused attention prologue uses, so both write the same bytes.
    float ssq = 0.0f;
    for (int i = lane * 8; i < HD; i += 64 * 8)
      ssq = ssq_f16x8(*reinterpret_cast<const u32x4*>(src + i), ssq);
    const float rstd = 1.0f / sqrtf(wave_sum(ssq) / (float)HD + eps);
    float xn[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) xn[i] = clip_qkv(h2f(f2h(h2f(f2h(xv[i] * rstd)) * wv[i])), clip, clip16);
    const bool first = lane < 32;  // d < D/2
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const float xs = __shfl_xor(xn[i], 32, 64);
      const float xr = first ? -xs : xs;
      o[i] = h2f(f2h(xn[i] * cv[i] + xr * sv[i]));
    }
    if (which == 0) {
#pragma unroll
      for (int i = 0; i < EPL; ++i) q_out[h * D + d0 + i] = f2h(o[i]);
      return;
    }
    if (k_rot_out) {
#pragma unroll
      for (int i = 0; i < EPL; ++i) k_rot_out[h * D + d0 + i] = f2h(o[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < EPL; ++i) o[i] = clip_qkv(xv[i], clip, clip16);
  }
  if (!pos_ok) return;
  // KV-INT8 quantisation of this head's row.
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) amax = fmaxf(amax, fabsf(o[i]));
  amax = wave_max(amax);
  const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
  int8_t* dst = (which == 1 ? kc : vc) + (int64_t)h * code_head_stride + pos * D;
  uint16_t* f16dst = which == 1 ? k_f16 : v_f16;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    float qv = rintf(o[i] / s);
    qv = fminf(fmaxf(qv, -127.0f), 127.0f);
    dst[d0 + i] = (int8_t)(int)qv;
    if (f16dst) f16dst[(int64_t)h * f16_head_stride + pos * D + d0 + i] = f2h(o[i]);
  }
  if (lane == 0) (which == 1 ? ks : vs)[(int64_t)h * s_len + pos] = f2h(s);
}

// Attention prologue of several prompt rows (prefill): one block per (row,
// part) with part 0 q, 1 k, 2 v; thread t holds the 8 elements
// [8t, 8t + 8) of the part's heads*D row (head 8t / D), so the RMSNorm over
// heads*D is one block reduction and the RoPE partner d +- D/2 sits D/16
// lanes away in the same wave.  q and k: q_norm/k_norm, then RoPE with HF's
// rounding (fp16(fp16(x*cos) + fp16(rotate_half(x)*sin))); k and v: the fp16
// row to the attention's cache and the KV-INT8 row (amax over the head's D/8
// threads).  Threads past heads*D/8 (a block is whole waves) only take part
// in the reductions, with zeros.
template <int D>
__global__ __launch_bounds__(1024) void qk_rows_kernel(
    const uint16_t* __restrict__ qkv, int HD, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, float eps, const uint16_t* __restrict__ cos_tab,
    const uint16_t* __restrict__ sin_tab, int64_t pos0, uint16_t* __restrict__ q_out,
    int8_t* __restrict__ kc, uint16_t* __restrict__ ks, int8_t* __restrict__ vc,
    uint16_t* __restrict__ vs, int64_t code_head_stride, int64_t s_len, uint16_t* __restrict__ k_f16,
    uint16_t* __restrict__ v_f16, int64_t f16_head_stride, float clip) {
  __shared__ float red[16];
  const float clip16 = h2f(f2h(clip));
  const int t = threadIdx.x, lane = t & 63;
  const int64_t row = blockIdx.x;
  const int part = blockIdx.y;
  const int64_t pos = pos0 + row;
  const bool active = 8 * t < HD;
  const int e0 = active ? 8 * t : 0;
  const int h = e0 / D, d0 = e0 % D;
  const uint16_t* src = qkv + row * 3 * HD + (int64_t)part * HD;
  const u32x4 raw = *reinterpret_cast<const u32x4*>(src + e0);
  const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
  float o[8];
  if (part < 2) {
    const uint16_t* nw = part == 0 ? qn_w : kn_w;
    const u32x4 wv = *reinterpret_cast<const u32x4*>(nw + e0);
    const u32x4 cv = *reinterpret_cast<const u32x4*>(cos_tab + pos * D + d0);
    const u32x4 sv = *reinterpret_cast<const u32x4*>(sin_tab + pos * D + d0);
    float ssq = active ? ssq_f16x8(raw, 0.0f) : 0.0f;
    ssq = wave_sum(ssq);
    if (lane == 0) red[t >> 6] = ssq;
    __syncthreads();
    float tot = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) tot += red[w];
    const float rstd = 1.0f / sqrtf(tot / (float)HD + eps);
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
    const uint32_t cw[4] = {cv.x, cv.y, cv.z, cv.w};
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
    const bool first = d0 < D / 2;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint16_t xb = (uint16_t)(rw[i / 2] >> (16 * (i & 1)));
      const uint16_t wb = (uint16_t)(ww[i / 2] >> (16 * (i & 1)));
      const float xn = clip_qkv(h2f(f2h(h2f(f2h(h2f(xb) * rstd)) * h2f(wb))), clip, clip16);
      const float xs = __shfl_xor(xn, D / 16, 64);
      const float c = h2f((uint16_t)(cw[i / 2] >> (16 * (i & 1))));
      const float sn = h2f((uint16_t)(sw[i / 2] >> (16 * (i & 1))));
      const float xr = first ? -xs : xs;
      {
        // Three roundings; without this pragma the compiler narrows the
        // products to fp16 multiplies and contracts one of them with the add
        // into a single-rounding fma.
#pragma clang fp contract(off)
        o[i] = h2f(f2h(h2f(f2h(xn * c)) + h2f(f2h(xr * sn))));
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = clip_qkv(h2f((uint16_t)(rw[i / 2] >> (16 * (i & 1)))), clip, clip16);
  }
  uint32_t packed[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) packed[i] = (uint32_t)f2h(o[2 * i]) | ((uint32_t)f2h(o[2 * i + 1]) << 16);
  const u32x4 ov = (u32x4){packed[0], packed[1], packed[2], packed[3]};
  if (part == 0) {
    if (active) *reinterpret_cast<u32x4*>(q_out + row * HD + e0) = ov;
    return;
  }
  uint16_t* fdst = part == 1 ? k_f16 : v_f16;
  if (!kc) {  // fp16 cache only (no KV-INT8 rows): a grid-uniform branch
    if (active) *reinterpret_cast<u32x4*>(fdst + (int64_t)h * f16_head_stride + pos * D + d0) = ov;
    return;
  }
  // KV-INT8 row of this head: amax over the head's D/8 threads
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(o[i]));
#pragma unroll
  for (int d = 1; d < D / 8; d <<= 1) amax = fmaxf(amax, __shfl_xor(amax, d, 64));
  const float sc = amax > 0.0f ? amax / 127.0f : 1.0f;
  uint32_t cw2[2] = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float qv = rintf(o[i] / sc);
    qv = fminf(fmaxf(qv, -127.0f), 127.0f);
    cw2[i / 4] |= ((uint32_t)(uint8_t)(int8_t)(int)qv) << (8 * (i % 4));
  }
  if (!active) return;
  int8_t* cdst = (part == 1 ? kc : vc) + (int64_t)h * code_head_stride + pos * D + d0;
  *reinterpret_cast<uint2*>(cdst) = make_uint2(cw2[0], cw2[1]);
  if (fdst) *reinterpret_cast<u32x4*>(fdst + (int64_t)h * f16_head_stride + pos * D + d0) = ov;
  if (d0 == 0) (part == 1 ? ks : vs)[(int64_t)h * s_len + pos] = f2h(sc);
}

}  // namespace

extern "C" int lemoq_rmsnorm(const uint16_t* x, int64_t rows, int64_t hidden, const uint16_t* w,
                             float eps, uint16_t* y, void* stream) {
  if (!x || !w || !y) return LEMOQ_ERR_NULL;
  if (rows < 0 || hidden <= 0 || hidden > 8192) return LEMOQ_ERR_SHAPE;
  if (rows == 0) return LEMOQ_OK;
  if (rows > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  const bool vec = hidden % 8 == 0 && hidden <= 2048 * RN_CHUNKS && lemoq_aligned16(x) && lemoq_aligned16(w) &&
                   lemoq_aligned16(y);
  if (vec)
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3((unsigned)rows), dim3(256), 0, lemoq_stream(stream), x,
                       (int)hidden, w, eps, y);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3((unsigned)rows), dim3(256), 0, lemoq_stream(stream), x,
                       (int)hidden, w, eps, y);
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_gather_rows(const uint16_t* src, int64_t n_rows, int64_t H, const int64_t* ids,
                                 int64_t rows, uint16_t* dst, void* stream) {
  if (!src || !ids || !dst) return LEMOQ_ERR_NULL;
  if (n_rows <= 0 || H <= 0 || H % 8 != 0 || rows < 0 || rows > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(src) || !lemoq_aligned16(dst)) return LEMOQ_ERR_ALIGN;
  if (rows == 0) return LEMOQ_OK;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)rows), dim3(256), 0, lemoq_stream(stream), src,
                     n_rows, H, ids, dst);
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_rope(const uint16_t* x, int64_t x_sh, int64_t x_sd, int64_t heads,
                          int64_t head_dim, const uint16_t* cos, const uint16_t* sin,
                          int64_t cs_sd, uint16_t* out, int64_t o_sh, int64_t o_sd,
                          void* stream) {
  if (!x || !cos || !sin || !out) return LEMOQ_ERR_NULL;
  if (heads <= 0 || heads > 65535 || head_dim < 2 || head_dim % 2 != 0 || head_dim > 1024)
    return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)heads), dim3(128), 0, lemoq_stream(stream), x,
                     x_sh, x_sd, (int)head_dim, cos, sin, cs_sd, out, o_sh, o_sd);
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_qk_norm_rope_kv_i8(const uint16_t* qkv, int64_t heads, int64_t head_dim,
                                        const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                                        float eps, const uint16_t* cos_tab,
                                        const uint16_t* sin_tab, const int64_t* pos,
                                        uint16_t* q_out, int8_t* kc, uint16_t* ks, int8_t* vc,
                                        uint16_t* vs, int64_t code_head_stride, int64_t s_len,
                                        uint16_t* k_f16, uint16_t* v_f16,
                                        int64_t f16_head_stride, uint16_t* k_rot_out,
                                        float clip_qkv, void* stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !pos || !q_out || !kc || !ks ||
      !vc || !vs)
    return LEMOQ_ERR_NULL;
  if (heads <= 0 || heads > 4096 || heads * head_dim > 65536) return LEMOQ_ERR_SHAPE;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return LEMOQ_ERR_UNSUPPORTED;
  if (!(clip_qkv >= 0.0f)) return LEMOQ_ERR_SHAPE;  // negative or NaN bound
  if (!lemoq_aligned16(qkv)) return LEMOQ_ERR_ALIGN;
  if (s_len <= 0 || code_head_stride < s_len * head_dim) return LEMOQ_ERR_SHAPE;
  if ((k_f16 || v_f16) && f16_head_stride < s_len * head_dim) return LEMOQ_ERR_SHAPE;
  const dim3 grid((unsigned)(3 * heads));
  hipStream_t st = lemoq_stream(stream);
#define LEMOQ_QK_CASE(EE)                                                                       \
  hipLaunchKernelGGL((qk_norm_rope_kv_kernel<EE>), grid, dim3(64), 0, st, qkv, (int)heads,     \
                     q_norm_w, k_norm_w, eps, cos_tab, sin_tab, pos, q_out, kc, ks, vc, vs,    \
                     code_head_stride, s_len, k_f16, v_f16, f16_head_stride, k_rot_out, clip_qkv);
  switch (head_dim) {
    case 64: LEMOQ_QK_CASE(1) break;
    case 128: LEMOQ_QK_CASE(2) break;
    default: LEMOQ_QK_CASE(4) break;
  }
#undef LEMOQ_QK_CASE
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_qk_norm_rope_kv_i8_rows(const uint16_t* qkv, int64_t rows, int64_t heads,
                                             int64_t head_dim, const uint16_t* q_norm_w,
                                             const uint16_t* k_norm_w, float eps,
                                             const uint16_t* cos_tab, const uint16_t* sin_tab,
                                             int64_t pos0, uint16_t* q_out, int8_t* kc,
                                             uint16_t* ks, int8_t* vc, uint16_t* vs,
                                             int64_t code_head_stride, int64_t s_len,
                                             uint16_t* k_f16, uint16_t* v_f16,
                                             int64_t f16_head_stride, float clip_qkv, void* stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !q_out) return LEMOQ_ERR_NULL;
  // KV-INT8 rows (all four buffers), or, with none of them, the fp16 rows only
  const bool i8 = kc || ks || vc || vs;
  if (i8 ? (!kc || !ks || !vc || !vs) : (!k_f16 || !v_f16)) return LEMOQ_ERR_NULL;
  if (heads <= 0 || heads > 4096 || heads * head_dim > 65536) return LEMOQ_ERR_SHAPE;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return LEMOQ_ERR_UNSUPPORTED;
  if (!(clip_qkv >= 0.0f)) return LEMOQ_ERR_SHAPE;  // negative or NaN bound
  if (!lemoq_aligned16(qkv)) return LEMOQ_ERR_ALIGN;
  if (s_len <= 0 || (i8 && code_head_stride < s_len * head_dim)) return LEMOQ_ERR_SHAPE;
  if ((k_f16 || v_f16) && f16_head_stride < s_len * head_dim) return LEMOQ_ERR_SHAPE;
  // every row's slot must exist: the cos/sin tables and the caches hold s_len positions
  if (rows <= 0 || rows > 0x7fffffffLL || pos0 < 0 || pos0 + rows > s_len) return LEMOQ_ERR_SHAPE;
  const int64_t HD = heads * head_dim;
  if (HD % 8 != 0 || HD / 8 > 1024) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(q_norm_w) || !lemoq_aligned16(k_norm_w) || !lemoq_aligned16(cos_tab) ||
      !lemoq_aligned16(sin_tab) || !lemoq_aligned16(q_out) || (k_f16 && !lemoq_aligned16(k_f16)) ||
      (v_f16 && !lemoq_aligned16(v_f16)) || (reinterpret_cast<uintptr_t>(kc) & 7u) ||
      (reinterpret_cast<uintptr_t>(vc) & 7u) || code_head_stride % 8 != 0 || f16_head_stride % 8 != 0)
    return LEMOQ_ERR_ALIGN;
  const unsigned threads = (unsigned)(((HD / 8) + 63) / 64 * 64);
  const dim3 grid((unsigned)rows, 3u);
  hipStream_t st = lemoq_stream(stream);
#define LEMOQ_QK_ROWS_CASE(DD)                                                                  \
  hipLaunchKernelGGL((qk_rows_kernel<DD>), grid, dim3(threads), 0, st, qkv, (int)HD, q_norm_w,   \
                     k_norm_w, eps, cos_tab, sin_tab, pos0, q_out, kc, ks, vc, vs,              \
                     code_head_stride, s_len, k_f16, v_f16, f16_head_stride, clip_qkv);
  switch (head_dim) {
    case 64: LEMOQ_QK_ROWS_CASE(64) break;
    case 128: LEMOQ_QK_ROWS_CASE(128) break;
    default: LEMOQ_QK_ROWS_CASE(256) break;
  }
#undef LEMOQ_QK_ROWS_CASE
  LEMOQ_CHECK_LAUNCH();
}
