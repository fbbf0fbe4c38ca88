// Quantisation and KV-cache write kernels: per-group RTN w8 (weights) and
// per-token symmetric int8 (KV cache), plus the bitwise fp16 KV slot write.
//
// Bit-exactness: the fp32 divisions below are IEEE correctly rounded (hipcc's
// default for `/` on float), rintf is v_rndne_f32 (round half to even, the
// rounding of torch.round / numpy.round) and the fp32 -> fp16 scale cast is
// round-to-nearest-even, so codes and scales reproduce the reference's torch
// arithmetic bit for bit.
#include "common.h"

// ---------------------------------------------------------------------------
// RTN w8, symmetric, per (row, group).  One wave per group; a block of 4
// waves covers 4 consecutive groups of one row.
// Reference arithmetic: src/lemoq/quant/rtn.py:68-73 (torch) and
// src/lemoq/quant/numpy_oracle.py:89-94 (numpy): scale = absmax / 127 in fp32
// (1.0 when absmax == 0), codes = round(w / scale).clamp(-128, 127).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rtn_w8_kernel(const float* __restrict__ w, int64_t rows,
                                                     int64_t cols, int64_t group,
                                                     int64_t n_groups,
                                                     int8_t* __restrict__ codes,
                                                     uint16_t* __restrict__ scale16,
                                                     float* __restrict__ scale32) {
  const int lane = threadIdx.x & 63;
  const int64_t gid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (row, group) index
  if (gid >= rows * n_groups) return;
  const int64_t row = gid / n_groups;
  const int64_t g = gid - row * n_groups;
  const int64_t padded = n_groups * group;
  const float* wr = w + row * cols;
  const int64_t k0 = g * group;

  float amax = 0.0f;
  for (int64_t i = lane; i < group; i += 64) {
    const int64_t k = k0 + i;
    const float v = k < cols ? wr[k] : 0.0f;
    amax = fmaxf(amax, fabsf(v));
  }
  amax = wave_max(amax);
  const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
  for (int64_t i = lane; i < group; i += 64) {
    const int64_t k = k0 + i;
    const float v = k < cols ? wr[k] : 0.0f;
    float q = rintf(v / s);
    q = fminf(fmaxf(q, -128.0f), 127.0f);
    codes[row * padded + k] = (int8_t)(int)q;
  }
  if (lane == 0) {
    scale16[gid] = f2h(s);
    if (scale32) scale32[gid] = s;
  }
}

extern "C" int lemoq_rtn_quantize_w8(const float* w, int64_t rows, int64_t cols, int64_t group,
                                     int8_t* codes, uint16_t* scale_f16, float* scale_f32,
                                     void* stream) {
  if (!w || !codes || !scale_f16) return LEMOQ_ERR_NULL;
  if (rows < 0 || cols <= 0 || group <= 0) return LEMOQ_ERR_SHAPE;
  if (rows == 0) return LEMOQ_OK;
  const int64_t n_groups = (cols + group - 1) / group;
  const int64_t total = rows * n_groups;
  const int64_t blocks = (total + 3) / 4;
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(rtn_w8_kernel, dim3((unsigned)blocks), dim3(256), 0, lemoq_stream(stream), w,
                     rows, cols, group, n_groups, codes, scale_f16, scale_f32);
  LEMOQ_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------
// Per-token symmetric int8 of one row of D fp16 values, one wave per row.
// Reference arithmetic: src/lemoq/kernels/kv_int8.py:30-41 (quantize_per_token_int8)
// and the write kernels :196-217, :294-312: amax in fp32, s = amax / 127
// (1.0 when amax == 0), q = rint(x / s) clamped to [-127, 127], scale -> fp16.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void quant_row_wave(const uint16_t* __restrict__ x, int D,
                                               int8_t* __restrict__ codes,
                                               uint16_t* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  float amax = 0.0f;
  for (int d = lane; d < D; d += 64) amax = fmaxf(amax, fabsf(h2f(x[d])));
  amax = wave_max(amax);
  const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
  for (int d = lane; d < D; d += 64) {
    float q = rintf(h2f(x[d]) / s);
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    codes[d] = (int8_t)(int)q;
  }
  if (lane == 0) *scale = f2h(s);
}

// grid = 2*heads waves (k rows then v rows), 4 waves per block.
__global__ __launch_bounds__(256) void kv_write_i8_kernel(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int heads, int D,
    int8_t* __restrict__ kc, uint16_t* __restrict__ ks, int8_t* __restrict__ vc,
    uint16_t* __restrict__ vs, int64_t code_head_stride, int64_t s_len,
    const int64_t* __restrict__ pos) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= 2 * heads) return;
  const int64_t slot = pos ? pos[0] : 0;
  if (slot < 0 || slot >= s_len) return;  // a position outside the cache writes nothing
  const bool is_k = r < heads;
  const int h = is_k ? r : r - heads;
  const uint16_t* src = (is_k ? k : v) + (int64_t)h * D;
  int8_t* dst = (is_k ? kc : vc) + (int64_t)h * code_head_stride + slot * D;
  uint16_t* sdst = (is_k ? ks : vs) + (int64_t)h * s_len + slot;
  quant_row_wave(src, D, dst, sdst);
}

extern "C" int lemoq_kv_write_i8(const uint16_t* k, const uint16_t* v, int64_t heads,
                                 int64_t head_dim, int8_t* kc, uint16_t* ks, int8_t* vc,
                                 uint16_t* vs, int64_t code_head_stride, int64_t s_len,
                                 const int64_t* pos, void* stream) {
  if (!k || !v || !kc || !ks || !vc || !vs) return LEMOQ_ERR_NULL;
  if (heads <= 0 || head_dim <= 0 || head_dim > 4096 || heads > 65536) return LEMOQ_ERR_SHAPE;
  if (code_head_stride < head_dim || s_len < 1) return LEMOQ_ERR_SHAPE;
  if (pos && code_head_stride < s_len * head_dim) return LEMOQ_ERR_SHAPE;
  const int rows = (int)(2 * heads);
  hipLaunchKernelGGL(kv_write_i8_kernel, dim3((rows + 3) / 4), dim3(256), 0, lemoq_stream(stream),
                     k, v, (int)heads, (int)head_dim, kc, ks, vc, vs, code_head_stride, s_len, pos);
  LEMOQ_CHECK_LAUNCH();
}

__global__ __launch_bounds__(256) void quantize_rows_kernel(const uint16_t* __restrict__ x,
                                                            int64_t rows, int D,
                                                            int8_t* __restrict__ codes,
                                                            uint16_t* __restrict__ scales) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  quant_row_wave(x + r * D, D, codes + r * D, scales + r);
}

extern "C" int lemoq_kv_quantize_rows(const uint16_t* x, int64_t rows, int64_t head_dim,
                                      int8_t* codes, uint16_t* scales, void* stream) {
  if (!x || !codes || !scales) return LEMOQ_ERR_NULL;
  if (rows < 0 || head_dim <= 0 || head_dim > 4096) return LEMOQ_ERR_SHAPE;
  if (rows == 0) return LEMOQ_OK;
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     lemoq_stream(stream), x, rows, (int)head_dim, codes, scales);
  LEMOQ_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------
// Bitwise fp16 KV slot write, one block per (k|v, head).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void kv_write_f16_kernel(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t src_head_stride,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, int64_t dst_head_stride,
    const int64_t* __restrict__ pos, int heads, int D) {
  const int r = blockIdx.x;
  const bool is_k = r < heads;
  const int h = is_k ? r : r - heads;
  const int64_t slot = pos[0];
  if (slot < 0 || (slot + 1) * D > dst_head_stride) return;  // outside the cache: no write
  const uint16_t* src = (is_k ? k : v) + (int64_t)h * src_head_stride;
  uint16_t* dst = (is_k ? k_cache : v_cache) + (int64_t)h * dst_head_stride + slot * D;
  for (int d = threadIdx.x; d < D; d += 64) dst[d] = src[d];
}

extern "C" int lemoq_kv_write_f16(const uint16_t* k, const uint16_t* v, int64_t src_head_stride,
                                  uint16_t* k_cache, uint16_t* v_cache, int64_t dst_head_stride,
                                  const int64_t* pos, int64_t heads, int64_t head_dim,
                                  void* stream) {
  if (!k || !v || !k_cache || !v_cache || !pos) return LEMOQ_ERR_NULL;
  if (heads <= 0 || heads > 65536 || head_dim <= 0 || src_head_stride < head_dim ||
      dst_head_stride < head_dim)
    return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(kv_write_f16_kernel, dim3((unsigned)(2 * heads)), dim3(64), 0,
                     lemoq_stream(stream), k, v, src_head_stride, k_cache, v_cache,
                     dst_head_stride, pos, (int)heads, (int)head_dim);
  LEMOQ_CHECK_LAUNCH();
}

// ---------------------------------------------------------------------------
extern "C" const char* lemoq_status_string(int status) {
  switch (status) {
    case LEMOQ_OK: return "ok";
    case LEMOQ_ERR_NULL: return "a required pointer is NULL";
    case LEMOQ_ERR_SHAPE: return "a size is out of range or inconsistent";
    case LEMOQ_ERR_UNSUPPORTED: return "the request is not supported by this build";
    case LEMOQ_ERR_ALIGN: return "a pointer is not 16-byte aligned";
    case LEMOQ_ERR_CAPACITY: return "the request exceeds a fixed capacity of the library";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown lemoq status";
}

extern "C" int lemoq_abi_version(void) { return LEMOQ_ABI_VERSION; }
