// Fused per-layer attention of the decode step over the KV-INT8 or the fp16
// cache, as one launch of split blocks (the block itself is in attn_fused.h).
#include "attn_fused.h"

namespace {

using lemoq_attn_fused::AttnSplitArgs;

template <int D, int NW_ = 8, int U_ = 4>
__global__ __launch_bounds__(64 * NW_) void attn_split_fused_i8_kernel(const AttnSplitArgs a) {
  __shared__ lemoq_attn_fused::AttnFusedSmem<D, NW_, 1> sm;
  lemoq_attn_fused::attn_split_fused_block<D, true, NW_, U_>(a, blockIdx.x, blockIdx.y, sm);
}

template <int D, int NW_ = 8, int U_ = 4>
__global__ __launch_bounds__(64 * NW_) void attn_split_fused_f16_kernel(const AttnSplitArgs a) {
  __shared__ lemoq_attn_fused::AttnFusedSmem<D, NW_, 2> sm;
  lemoq_attn_fused::attn_split_fused_block<D, false, NW_, U_>(a, blockIdx.x, blockIdx.y, sm);
}

// The rules both cache kinds share; the fp16 cache passes no scales.
int check_fused(const uint16_t* qkv, int64_t heads, int64_t head_dim, const uint16_t* q_norm_w,
                const uint16_t* k_norm_w, const uint16_t* cos_tab, const uint16_t* sin_tab,
                const int64_t* pos, const void* kc, const void* vc, int64_t code_head_stride,
                int64_t s_len, int64_t num_splits, const float* m, const float* l, const float* acc,
                float clip_qkv, int eb) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !pos || !kc || !vc || !m || !l ||
      !acc)
    return LEMOQ_ERR_NULL;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return LEMOQ_ERR_UNSUPPORTED;
  if (heads <= 0 || heads > 65535 || heads * head_dim > 65536) return LEMOQ_ERR_SHAPE;
  if (num_splits <= 0 || num_splits > 65535) return LEMOQ_ERR_SHAPE;
  if (!(clip_qkv >= 0.0f)) return LEMOQ_ERR_SHAPE;  // negative or NaN bound
  if (s_len <= 0 || s_len >= (int64_t(1) << 31) || code_head_stride < s_len * head_dim)
    return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(qkv) || !lemoq_aligned16(kc) || !lemoq_aligned16(vc) ||
      (code_head_stride * eb) % 16 != 0)
    return LEMOQ_ERR_ALIGN;
  return LEMOQ_OK;
}

AttnSplitArgs fused_args(const uint16_t* qkv, int64_t heads, const uint16_t* q_norm_w,
                         const uint16_t* k_norm_w, float eps, const uint16_t* cos_tab,
                         const uint16_t* sin_tab, const int64_t* pos, void* kc, uint16_t* ks,
                         void* vc, uint16_t* vs, int64_t code_head_stride, int64_t s_len,
                         int64_t num_splits, float qk_scale, float* m, float* l, float* acc,
                         float clip_qkv) {
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
  a.clip = clip_qkv;
  a.m_out = m;
  a.l_out = l;
  a.acc_out = acc;
  return a;
}

}  // namespace

extern "C" int lemoq_attn_split_fused_i8(const uint16_t* qkv, int64_t heads, int64_t head_dim,
                                         const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                                         float eps, const uint16_t* cos_tab,
                                         const uint16_t* sin_tab, const int64_t* pos, int8_t* kc,
                                         uint16_t* ks, int8_t* vc, uint16_t* vs,
                                         int64_t code_head_stride, int64_t s_len,
                                         int64_t num_splits, float qk_scale, float* m, float* l,
                                         float* acc, float clip_qkv, void* stream) {
  if (!ks || !vs) return LEMOQ_ERR_NULL;
  const int rc = check_fused(qkv, heads, head_dim, q_norm_w, k_norm_w, cos_tab, sin_tab, pos, kc, vc,
                             code_head_stride, s_len, num_splits, m, l, acc, clip_qkv, 1);
  if (rc) return rc;
  const AttnSplitArgs a = fused_args(qkv, heads, q_norm_w, k_norm_w, eps, cos_tab, sin_tab, pos, kc, ks, vc,
                                     vs, code_head_stride, s_len, num_splits, qk_scale, m, l, acc, clip_qkv);
  hipStream_t st = lemoq_stream(stream);
  const dim3 grid((unsigned)num_splits, (unsigned)heads);
  // 4 waves per block (two blocks share a CU), 3 token loads per wave in
  // flight per token block: the fastest shape measured at 1 100 and 4 200
  // cache slots with 16 splits (against 8 and 16 waves, 1, 2 and 4 loads).
  const dim3 block(64 * 4);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL((attn_split_fused_i8_kernel<64, 4, 3>), grid, block, 0, st, a); break;
    case 128: hipLaunchKernelGGL((attn_split_fused_i8_kernel<128, 4, 3>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((attn_split_fused_i8_kernel<256, 4, 3>), grid, block, 0, st, a); break;
  }
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_attn_split_fused_f16(const uint16_t* qkv, int64_t heads, int64_t head_dim,
                                          const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                                          float eps, const uint16_t* cos_tab,
                                          const uint16_t* sin_tab, const int64_t* pos, uint16_t* kc,
                                          uint16_t* vc, int64_t head_stride, int64_t s_len,
                                          int64_t num_splits, float qk_scale, float* m, float* l,
                                          float* acc, float clip_qkv, void* stream) {
  const int rc = check_fused(qkv, heads, head_dim, q_norm_w, k_norm_w, cos_tab, sin_tab, pos, kc, vc,
                             head_stride, s_len, num_splits, m, l, acc, clip_qkv, 2);
  if (rc) return rc;
  const AttnSplitArgs a = fused_args(qkv, heads, q_norm_w, k_norm_w, eps, cos_tab, sin_tab, pos, kc, nullptr,
                                     vc, nullptr, head_stride, s_len, num_splits, qk_scale, m, l, acc,
                                     clip_qkv);
  hipStream_t st = lemoq_stream(stream);
  const dim3 grid((unsigned)num_splits, (unsigned)heads);
  // 4 waves per block and 3 token loads per wave (12 tokens at D 128), as
  // for KV-INT8: in the OLMoE step, 2 / 3 / 4 / 6 / 8 loads gave 0.513 /
  // 0.504 / 0.520 / 0.513 / 0.517 ms at ctx 1024 and 0.582 / 0.572 / 0.589 /
  // 0.578 / 0.594 ms at ctx 4096.
  constexpr int U = 3;
  const dim3 block(64 * 4);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL((attn_split_fused_f16_kernel<64, 4, U>), grid, block, 0, st, a); break;
    case 128: hipLaunchKernelGGL((attn_split_fused_f16_kernel<128, 4, U>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((attn_split_fused_f16_kernel<256, 4, U>), grid, block, 0, st, a); break;
  }
  LEMOQ_CHECK_LAUNCH();
}
