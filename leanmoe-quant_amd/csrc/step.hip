// Native decode-step executor: enqueues one whole OLMoE decode step of the
// canonical cell (w8a16 attention + experts, W8 lm_head, KV-INT8 cache; or the
// fp16 cache with kv_fp16) on a stream, ready to be captured into a hipGraph
// by the caller.
//
// Per layer (6 launches):
//   1 gemv_w8_fused   input RMSNorm (+ embedding gather on layer 0) -> packed q|k|v
//   2 attn_split_fused q_norm/k_norm, RoPE at *pos, KV-INT8 (or fp16) write of
//                     slot *pos, split-KV partials over [0, *pos]
//   3 attn_merge_o_proj  LSE merge of each block's 4 heads + their share of
//                     o_proj -> fp32 partial sums per head group
//   4 router_logits_resid  o = fp16(sum of partials), h_mid = fp16(o + h),
//                     post-attention RMSNorm + router GEMV -> fp16 logits
//                     (one wave per expert row)
//   5 moe_gate_up_w8  softmax/top-k of the logits in every wave, then gate/up
//                     + SiLU of the 8 selected experts (stores ids, weights)
//   6 moe_down_w8     down projection x routing weight + residual (h_mid) -> h
// Shapes outside the fused attention-output path (or a step without o_part /
// h_mid) run 3-4 as three launches: attn_merge, the o_proj GEMV with the
// residual add in its epilogue, router_logits.
// then final RMSNorm + lm_head GEMV with per-block argmax partials, and the
// greedy selection that writes the next token and advances *pos / *filled.
//
// 4-bit weights (weight_bits 4, the reference's w4a16 cell) run the same
// layer on 4-bit kernels: the q|k|v GEMV with the input RMSNorm in its
// prologue, the same fused attention, merge + 4-bit o_proj (or, off the fused
// shape rule, the merge, the 4-bit o_proj GEMV with the residual add and the
// router logits), the routed 4-bit gate/up and the 4-bit down with the
// residual add; layer 0 first gathers the embedding row.  An fp16 lm_head (lm_f16, the reference's
// lm_head in every cell but w8a16 with its lm_head switch on) ends the step
// with the final norm + fp16 GEMV writing the argmax partials and the greedy
// selection over them, the W8 head's two launches.
//
// Every shape and buffer rule of every launch is checked before the first
// launch is enqueued, so a rejected step leaves the cache and buffers as they
// were.
//
// The layer order and rounding points restate the HF OLMoE decoder layer
// (transformers OlmoeDecoderLayer/OlmoeModel, called by the reference through
// StaticCacheDecodeSession, benchmarks/cudagraph.py:720-737) with the
// reference's patched operators (attn_decode.py:836-1017,
// moe_grouped_quant.py:562-601, rmsnorm.py:205-212).
#include "common.h"

#define LEMOQ_TRY(expr)       \
  do {                        \
    const int rc__ = (expr);  \
    if (rc__) return rc__;    \
  } while (0)

namespace {

bool a16(const void* p) { return lemoq_aligned16(p); }

bool overlaps(const void* x, int64_t nx, const void* y, int64_t ny) {
  const char* p = static_cast<const char*>(x);
  const char* q = static_cast<const char*>(y);
  return p < q + ny && q < p + nx;
}

// A w8 GEMV launch of the step: its weights' shape rules (gemv.hip).
int check_gemv(int64_t N, int64_t K, int64_t group) {
  if (N <= 0 || K <= 0) return LEMOQ_ERR_SHAPE;
  if (K > 8192 || K % 16 != 0 || K % group != 0) return LEMOQ_ERR_UNSUPPORTED;
  if ((N + 7) / 8 > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  return LEMOQ_OK;
}

enum AttnPath { kAttnFusedOut, kAttnThree };

// Every rule of every launch of the step, before anything is enqueued.
int validate(const LemoqOlmoeStep* p, AttnPath* path) {
  if (!p || !p->layers) return LEMOQ_ERR_NULL;
  if (p->kv_fp16 != 0 && p->kv_fp16 != 1) return LEMOQ_ERR_SHAPE;
  if (!p->embed || !p->final_norm || !p->cos_tab || !p->sin_tab || !p->token || !p->pos ||
      !p->filled || !p->h || !p->xn || !p->qkv || !p->q_rot || !p->attn || !p->part_m ||
      !p->part_l || !p->part_acc || !p->top_w || !p->top_i || !p->act || !p->logits ||
      !p->router_logits)
    return LEMOQ_ERR_NULL;
  // the argmax partials (either lm_head) and the W8 lm_head (not read with an fp16 lm_head)
  if (!p->am_val || !p->am_idx || (!p->lm_f16 && (!p->lm_codes || !p->lm_scale))) return LEMOQ_ERR_NULL;
  const int64_t H = p->hidden, D = p->head_dim, HD = p->heads * p->head_dim, E = p->num_experts;
  const int64_t F = p->ffn, K = p->top_k, g = p->group, S = p->max_seq, ns = p->num_splits;
  if (H <= 0 || p->heads <= 0 || D <= 0 || p->num_layers <= 0 || S <= 0 || ns <= 0 ||
      p->vocab <= 0 || E <= 0 || F <= 0 || K <= 0)
    return LEMOQ_ERR_SHAPE;
  if (g <= 0 || g % 16 != 0) return LEMOQ_ERR_UNSUPPORTED;
  if (!(p->clip_qkv >= 0.0f)) return LEMOQ_ERR_SHAPE;  // negative or NaN clip_qkv
  if (p->weight_bits != 8 && p->weight_bits != 4) return LEMOQ_ERR_UNSUPPORTED;
  const bool w4 = p->weight_bits == 4;
  // qkv GEMV (K = H), o_proj (K = HD) on the unfused path
  LEMOQ_TRY(check_gemv(3 * HD, H, g));
  if (p->vocab > 0x7ffffffeLL) return LEMOQ_ERR_SHAPE;
  if (p->am_len < lemoq_lm_head_argmax_parts(p->vocab)) return LEMOQ_ERR_SHAPE;
  if (p->lm_f16) {  // final norm + fp16 lm_head with the argmax partials (lemoq_lm_head_argmax_f16)
    if (H > 8192 || H % 16 != 0) return LEMOQ_ERR_UNSUPPORTED;
    if (!a16(p->lm_f16) || !a16(p->h) || !a16(p->final_norm)) return LEMOQ_ERR_ALIGN;
  } else {
    LEMOQ_TRY(check_gemv(p->vocab, H, g));
    if (!a16(p->lm_codes)) return LEMOQ_ERR_ALIGN;
  }
  if (w4) {
    // 4-bit GEMVs (lemoq_gemv_q rules), routed gate/up and down (moe_q4.hip),
    // row norm, gather, merge and router logits of the 4-bit layer
    if (g % 32 != 0 || HD > 8192 || HD % g != 0 || H % 32 != 0 || F % 32 != 0) return LEMOQ_ERR_UNSUPPORTED;
    if (ns > 1024) return LEMOQ_ERR_SHAPE;
    if (!a16(p->h) || !a16(p->embed) || !a16(p->attn)) return LEMOQ_ERR_ALIGN;
  }
  // split-KV attention (attn_fused.hip)
  if (D != 64 && D != 128 && D != 256) return LEMOQ_ERR_UNSUPPORTED;
  if (p->heads > 65535 || HD > 65536 || ns > 65535 || S >= ((int64_t)1 << 31)) return LEMOQ_ERR_SHAPE;
  if (!a16(p->qkv)) return LEMOQ_ERR_ALIGN;
  // routed gate/up and down (moe.hip)
  if (K > 64 || K > E) return LEMOQ_ERR_SHAPE;
  if (E > 256) return LEMOQ_ERR_UNSUPPORTED;
  if (F > 8192 || F % 16 != 0 || F % g != 0) return LEMOQ_ERR_UNSUPPORTED;
  if (E * 2 * F * H >= ((int64_t)1 << 40)) return LEMOQ_ERR_SHAPE;
  if (!a16(p->xn) || !a16(p->act)) return LEMOQ_ERR_ALIGN;
  for (int64_t L = 0; L < p->num_layers; ++L) {
    const LemoqOlmoeLayer& w = p->layers[L];
    if (!w.ln_in || !w.ln_post || !w.q_norm || !w.k_norm || !w.qkv_codes || !w.qkv_scale ||
        !w.o_codes || !w.o_scale || !w.router || !w.gu_codes || !w.gu_scale || !w.dn_codes ||
        !w.dn_scale || !w.kc || !w.vc || (!p->kv_fp16 && (!w.ks || !w.vs)))
      return LEMOQ_ERR_NULL;
    if (!a16(w.qkv_codes) || !a16(w.o_codes) || !a16(w.gu_codes) || !a16(w.dn_codes) || !a16(w.kc) ||
        !a16(w.vc) || !a16(w.router) || !a16(w.ln_post))
      return LEMOQ_ERR_ALIGN;
  }
  // the attention-output half: two launches (merge + o_proj, residual + norm +
  // router) or three (merge, o_proj with the residual, norm + router)
  const int64_t n_part = HD / 512;
  const bool fused_o = p->o_part && p->h_mid && D == 128 && p->heads % 4 == 0 && ns <= 64 &&
                       (H == 2048 || H == 4096) &&
                       (n_part == 1 || n_part == 2 || n_part == 4 || n_part == 8) && HD % g == 0 &&
                       H % 32 == 0 && E <= 4 * 65535;
  if (fused_o) {
    if (!a16(p->o_part) || !a16(p->h_mid) || !a16(p->h)) return LEMOQ_ERR_ALIGN;
    if (overlaps(p->h_mid, H * 2, p->h, H * 2) || overlaps(p->h_mid, H * 2, p->o_part, n_part * H * 4))
      return LEMOQ_ERR_SHAPE;
    *path = kAttnFusedOut;
  } else {
    LEMOQ_TRY(check_gemv(H, HD, g));  // the o_proj GEMV (w8, or the 4-bit rules checked above)
    if (ns > 1024 || D > 256) return LEMOQ_ERR_SHAPE;
    if (H > 8192 || H % 16 != 0) return LEMOQ_ERR_UNSUPPORTED;
    if (E > 65536) return LEMOQ_ERR_SHAPE;
    if (!a16(p->attn)) return LEMOQ_ERR_ALIGN;
    *path = kAttnThree;
  }
  return LEMOQ_OK;
}

}  // namespace

namespace {

// Split-KV attention of one layer: q/k norm, RoPE, cache write at slot *pos,
// partials over [0, *pos].
int enqueue_attention(const LemoqOlmoeStep* p, const LemoqOlmoeLayer& w, void* stream) {
  const int64_t D = p->head_dim, S = p->max_seq;
  if (p->kv_fp16)
    return lemoq_attn_split_fused_f16(p->qkv, p->heads, D, w.q_norm, w.k_norm, p->eps, p->cos_tab, p->sin_tab,
                                      p->pos, reinterpret_cast<uint16_t*>(w.kc),
                                      reinterpret_cast<uint16_t*>(w.vc), S * D, S, p->num_splits, p->qk_scale,
                                      p->part_m, p->part_l, p->part_acc, p->clip_qkv, stream);
  return lemoq_attn_split_fused_i8(p->qkv, p->heads, D, w.q_norm, w.k_norm, p->eps, p->cos_tab, p->sin_tab,
                                   p->pos, w.kc, w.ks, w.vc, w.vs, S * D, S, p->num_splits, p->qk_scale,
                                   p->part_m, p->part_l, p->part_acc, p->clip_qkv, stream);
}

// Final norm + lm_head and the greedy selection / step advance.
int enqueue_head(const LemoqOlmoeStep* p, void* stream) {
  const int64_t H = p->hidden;
  if (p->lm_f16)
    return lemoq_lm_head_argmax_f16(p->h, p->final_norm, p->eps, p->lm_f16, p->vocab, H, p->logits, p->am_val,
                                    p->am_idx, p->am_len, p->token, p->pos, p->filled, p->prompt, p->prompt_len,
                                    p->history, p->history_len, stream);
  return lemoq_lm_head_argmax_w8(p->h, p->final_norm, p->eps, p->lm_codes, p->lm_scale, p->vocab, H,
                                 p->group, p->logits, p->am_val, p->am_idx, p->am_len, p->token, p->pos,
                                 p->filled, p->prompt, p->prompt_len, p->history, p->history_len, stream);
}

// Whether the 4-bit q|k|v GEMV normalises once per block (lemoq_gemv_q_rmsnorm's
// rule: 4-bit rows of H codes fill its 1 KB chunks exactly for H 2048, 4096,
// 8192; the step's buffers are 16-byte aligned), which lets it gather layer
// 0's embedding row itself.
bool qkv_w4_block_norm(const LemoqOlmoeStep* p) {
  const int64_t H = p->hidden;
  return (H == 2048 || H == 4096 || H == 8192) && a16(p->embed) && a16(p->h) && a16(p->layers[0].ln_in);
}

// One layer on 4-bit weights: 6 launches on the fused attention-output path,
// 7 otherwise (plus, on layer 0, the embedding gather when the q|k|v GEMV
// cannot do it).
int enqueue_layer_w4(const LemoqOlmoeStep* p, const LemoqOlmoeLayer& w, bool first, AttnPath path, void* stream) {
  const int64_t H = p->hidden, HD = p->heads * p->head_dim, g = p->group;
  // input RMSNorm + packed q|k|v; layer 0 gathers the embedding row of *token and
  // stores it as the residual (in the GEMV when it takes the per-block norm)
  const bool gather_in_gemv = qkv_w4_block_norm(p);
  if (first && !gather_in_gemv) LEMOQ_TRY(lemoq_gather_rows(p->embed, p->vocab, H, p->token, 1, p->h, stream));
  const bool g0 = first && gather_in_gemv;
  LEMOQ_TRY(lemoq_gemv_q_rmsnorm(g0 ? p->embed : p->h, g0 ? p->token : nullptr, g0 ? p->vocab : 0, 1, H, w.ln_in,
                                 p->eps, g0 ? p->h : nullptr, w.qkv_codes, LEMOQ_QFMT_W4, w.qkv_scale, nullptr, 0,
                                 3 * HD, H, g, p->qkv, 1, stream));
  LEMOQ_TRY(enqueue_attention(p, w, stream));
  if (path == kAttnFusedOut) {
    // LSE merge + 4-bit o_proj partials per group of 4 heads; h_mid = fp16(fp16(o) + h),
    // post-attention RMSNorm + router logits
    LEMOQ_TRY(lemoq_attn_merge_o_proj_w4(p->part_m, p->part_l, p->part_acc, p->heads, p->num_splits,
                                         p->head_dim, reinterpret_cast<const uint8_t*>(w.o_codes), w.o_scale, H,
                                         g, p->o_part, stream));
    LEMOQ_TRY(lemoq_router_logits_resid(p->o_part, HD / 512, p->h, w.ln_post, p->eps, H, w.router,
                                        p->num_experts, p->h_mid, p->xn, p->router_logits, stream));
  } else {
    LEMOQ_TRY(lemoq_attn_merge(p->part_m, p->part_l, p->part_acc, p->heads, p->num_splits, p->head_dim,
                               p->attn, stream));
    // o_proj; h = fp16(fp16(o) + h)
    LEMOQ_TRY(lemoq_gemv_q_residual(p->attn, 1, HD, w.o_codes, LEMOQ_QFMT_W4, w.o_scale, nullptr, 0, H, HD, g,
                                    p->h, p->h, stream));
    LEMOQ_TRY(lemoq_router_logits(p->h, w.ln_post, p->eps, H, w.router, p->num_experts, p->xn,
                                  p->router_logits, stream));
  }
  const uint16_t* resid = path == kAttnFusedOut ? p->h_mid : p->h;
  LEMOQ_TRY(lemoq_moe_gate_up_w4_routed(p->xn, reinterpret_cast<const uint8_t*>(w.gu_codes), w.gu_scale,
                                        p->router_logits, p->top_k, (int)p->norm_topk_prob, p->num_experts,
                                        p->ffn, H, g, p->act, p->top_i, p->top_w, stream));
  return lemoq_moe_down_w4(p->act, reinterpret_cast<const uint8_t*>(w.dn_codes), w.dn_scale, p->top_i, p->top_w,
                           p->top_k, p->num_experts, H, p->ffn, g, resid, p->h, stream);
}

}  // namespace

extern "C" int lemoq_olmoe_decode_step(const LemoqOlmoeStep* p, void* stream) {
  AttnPath path = kAttnThree;
  LEMOQ_TRY(validate(p, &path));
  if (p->weight_bits == 4) {
    for (int64_t L = 0; L < p->num_layers; ++L)
      LEMOQ_TRY(enqueue_layer_w4(p, p->layers[L], L == 0, path, stream));
    return enqueue_head(p, stream);
  }
  const int64_t H = p->hidden, HD = p->heads * p->head_dim, D = p->head_dim;
  const int64_t n_part = HD / 512;
  for (int64_t L = 0; L < p->num_layers; ++L) {
    const LemoqOlmoeLayer& w = p->layers[L];
    const bool first = L == 0;
    // 1. input RMSNorm + packed qkv projection.  Layer 0 gathers the
    //    embedding row of *token and block 0 stores it as the residual.
    LEMOQ_TRY(lemoq_gemv_w8_fused(first ? p->embed : p->h, first ? p->token : nullptr, p->vocab,
                                  w.ln_in, p->eps, first ? p->h : nullptr, w.qkv_codes,
                                  w.qkv_scale, 3 * HD, H, p->group, nullptr, p->qkv, stream));
    // 2. q/k norm, RoPE, cache write at slot *pos, split-KV partials.
    LEMOQ_TRY(enqueue_attention(p, w, stream));
    if (path == kAttnFusedOut) {
      // 3. LSE merge + o_proj partials per group of 4 heads.
      LEMOQ_TRY(lemoq_attn_merge_o_proj_w8(p->part_m, p->part_l, p->part_acc, p->heads,
                                           p->num_splits, D, w.o_codes, w.o_scale, H, p->group,
                                           p->o_part, stream));
      // 4. h_mid = fp16(fp16(o) + h); post-attention RMSNorm + router logits.
      LEMOQ_TRY(lemoq_router_logits_resid(p->o_part, n_part, p->h, w.ln_post, p->eps, H,
                                          w.router, p->num_experts, p->h_mid, p->xn,
                                          p->router_logits, stream));
    } else {
      // 3. LSE merge of the partials.
      LEMOQ_TRY(lemoq_attn_merge(p->part_m, p->part_l, p->part_acc, p->heads, p->num_splits, D,
                                 p->attn, stream));
      // 4. o_proj; h = fp16(fp16(o) + h).
      LEMOQ_TRY(lemoq_gemv_w8_fused(p->attn, nullptr, 0, nullptr, p->eps, nullptr, w.o_codes,
                                    w.o_scale, H, HD, p->group, p->h, p->h, stream));
      // 4b. post-attention RMSNorm + router logits.
      LEMOQ_TRY(lemoq_router_logits(p->h, w.ln_post, p->eps, H, w.router, p->num_experts, p->xn,
                                    p->router_logits, stream));
    }
    const uint16_t* resid = path == kAttnFusedOut ? p->h_mid : p->h;
    // 5-6. routing + grouped MoE; h = fp16(fp16(moe) + residual).
    LEMOQ_TRY(lemoq_moe_gate_up_w8_routed(p->xn, w.gu_codes, w.gu_scale, p->router_logits,
                                          p->top_k, (int)p->norm_topk_prob, p->num_experts,
                                          p->ffn, H, p->group, p->act, p->top_i, p->top_w,
                                          stream));
    LEMOQ_TRY(lemoq_moe_down_w8(p->act, w.dn_codes, w.dn_scale, p->top_i, p->top_w, p->top_k,
                                p->num_experts, H, p->ffn, p->group, resid, p->h, stream));
  }
  // Final norm + lm_head (W8 with argmax partials, or fp16), then greedy selection and step advance.
  return enqueue_head(p, stream);
}
