/*
 * lemoq_hip.h — C-ABI of the MI355X (gfx950) kernels behind the lemoq batch-1
 * OLMoE decode path: w8a16 grouped MoE, w8 dense GEMV, split-KV attention
 * (fp16 and KV-INT8) with its log-sum-exp merge, RMSNorm, RoPE, router top-k
 * and the KV write kernels.
 *
 * Conventions shared by every entry point:
 *   - Plain pointers and sizes only.  fp16 data is passed as uint16_t (IEEE
 *     binary16 bit patterns); int8 codes as int8_t; device scalars that the
 *     kernels read at run time (positions, filled lengths, expert ids, token
 *     ids) are device pointers, never host integers, so a captured hipGraph
 *     stays valid while they change.
 *   - `stream` is a hipStream_t passed as an opaque pointer (NULL = the null
 *     stream).  Every call only enqueues work: no host synchronisation, no
 *     device->host reads, no allocation or free of any memory.  Outputs and
 *     workspaces are caller-owned.
 *   - Return value: 0 on success; a negative LEMOQ_ERR_* code when the
 *     arguments are rejected before anything is launched; a positive value is
 *     the hipError_t reported by the launch.  lemoq_status_string() names it.
 *   - All entry points are stateless and reentrant, except
 *     lemoq_gemm_f16_splitk_noalloc, whose calls on one device share a fixed
 *     library-owned array (see its declaration).
 *
 * Reference interfaces replaced are cited as path:line into LeanMoE-Quant.
 */
#ifndef LEMOQ_HIP_H
#define LEMOQ_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LEMOQ_ABI_VERSION 8

enum {
  LEMOQ_OK = 0,
  LEMOQ_ERR_NULL = -1,        /* a required pointer is NULL                  */
  LEMOQ_ERR_SHAPE = -2,       /* a size is out of range or inconsistent      */
  LEMOQ_ERR_UNSUPPORTED = -3, /* a valid request this build does not cover   */
  LEMOQ_ERR_ALIGN = -4,       /* a pointer is not 16-byte aligned            */
  LEMOQ_ERR_CAPACITY = -5     /* larger than a fixed capacity of the library */
};

/* Human-readable name of a status returned by any lemoq_* call. */
const char* lemoq_status_string(int status);
/* LEMOQ_ABI_VERSION of the loaded library. */
int lemoq_abi_version(void);

/* ---------------------------------------------------------------------------
 * A2 — per-group symmetric RTN, 8-bit.
 * Replaces lemoq.quant.rtn.quantize_rtn (src/lemoq/quant/rtn.py:38-99) for
 * bits=8, symmetric=True, and the fp16 scale cast done by
 * quantize_fused_experts (src/lemoq/kernels/moe_grouped_quant.py:222-233) and
 * QuantLinear (src/lemoq/quant/linear.py:332).
 * w (rows, cols) fp32 row-major; groups of `group` along cols, the last group
 * zero-padded to padded = ceil(cols/group)*group.  Writes codes (rows, padded)
 * int8 and, per (row, group), scale_f16 (fp16 of the fp32 scale) and, when
 * non-NULL, scale_f32.  scale = absmax/127 (1.0 when absmax == 0), codes =
 * round-half-even(w/scale) clamped to [-128, 127], both in fp32.
 * ------------------------------------------------------------------------- */
int lemoq_rtn_quantize_w8(const float* w, int64_t rows, int64_t cols, int64_t group,
                          int8_t* codes, uint16_t* scale_f16, float* scale_f32,
                          void* stream);

/* ---------------------------------------------------------------------------
 * Weight formats of the dense dequant operator (the `bits`, `symmetric`,
 * `zero` and `mxfp4` arguments of dequant_gemm_fused,
 * src/lemoq/kernels/_dequant_triton.py:155-293, and the schemes of
 * QuantLinear, src/lemoq/quant/linear.py:76-89):
 *   LEMOQ_QFMT_W8       int8 codes, w = c * s                 (N, padded_k) bytes
 *   LEMOQ_QFMT_W8_ASYM  uint8 codes, w = (c - z) * s          (N, padded_k) bytes
 *   LEMOQ_QFMT_W4       int4 codes (-8..7), w = c * s         (N, padded_k / 2)
 *   LEMOQ_QFMT_W4_ASYM  uint4 codes (0..15), w = (c - z) * s  (N, padded_k / 2)
 *   LEMOQ_QFMT_MXFP4    E2M1 codes (bit 3 sign, bits 2..0 the magnitude
 *                       0, 0.5, 1, 1.5, 2, 3, 4, 6), w = e2m1(c) * 2^(X - 127)
 *                       with X the E8M0 scale byte of each 32 codes  (N, padded_k / 2)
 * 4-bit codes are two per byte, the even column in the low nibble
 * (src/lemoq/quant/pack.py:21-37).  Scales and zero points are per (row,
 * group of `group` codes along k): fp16 (scale_is_f32 = 0) or fp32, the zero
 * points of the same type; MXFP4 scales are uint8 E8M0 bytes with group 32 and
 * no zero point.
 * ------------------------------------------------------------------------- */
enum {
  LEMOQ_QFMT_W8 = 0,
  LEMOQ_QFMT_W8_ASYM = 1,
  LEMOQ_QFMT_W4 = 2,
  LEMOQ_QFMT_W4_ASYM = 3,
  LEMOQ_QFMT_MXFP4 = 4
};

/* Per-group RTN at 4 or 8 bits, symmetric or asymmetric.  Replaces
 * lemoq.quant.rtn.quantize_rtn (src/lemoq/quant/rtn.py:38-99) and, for 4
 * bits, pack.pack_4bit of its padded codes (src/lemoq/quant/pack.py:21-37).
 * w (rows, cols) fp32; padded = ceil(cols / group) * group (group even at 4
 * bits).  codes: (rows, padded) int8 (8-bit symmetric) or uint8 (8-bit
 * asymmetric), or (rows, padded / 2) packed bytes (4-bit).  Per (row, group),
 * each output that is non-NULL: scale_f16 / scale_f32 and zero_f16 / zero_f32
 * (zero 0 when symmetric).  Symmetric: s = absmax / qmax (1 for an all-zero
 * group), c = clamp(rint(w / s), -qmax - 1, qmax), qmax = 2^(bits-1) - 1.
 * Asymmetric, over the real columns only: s = (max - min) / qmax (1 when
 * max == min), z = rint(-min / s), c = clamp(rint(w / s) + z, 0, qmax),
 * qmax = 2^bits - 1.  fp32 arithmetic, IEEE division, round half to even. */
int lemoq_rtn_quantize(const float* w, int64_t rows, int64_t cols, int64_t group, int bits,
                       int symmetric, uint8_t* codes, uint16_t* scale_f16, float* scale_f32,
                       uint16_t* zero_f16, float* zero_f32, void* stream);

/* MXFP4 quantiser.  Replaces lemoq.quant.mxfp4.quantize_mxfp4
 * (src/lemoq/quant/mxfp4.py:50-102).  w (rows, cols) fp32; columns padded
 * with zeros to nblk * 32.  codes_packed (rows, nblk * 16) bytes,
 * scale_e8m0 (rows, nblk).  Per block: X = clamp(floor(log2(amax)) - 2, -127,
 * 127) (-127 for an all-zero block; log2 rounded to fp32 as torch's is),
 * byte X + 127; v = w / 2^X; the magnitude code is the first nearest of
 * {0, 0.5, 1, 1.5, 2, 3, 4, 6} to min(|v|, 6); the sign bit is v < 0. */
int lemoq_mxfp4_quantize(const float* w, int64_t rows, int64_t cols, uint8_t* codes_packed,
                         uint8_t* scale_e8m0, void* stream);

/* Decode GEMV over any LEMOQ_QFMT_* weight: y (M, N) = x (M, K) @ w^T with w
 * as above in fp32 and fp32 accumulation (the fused arm,
 * src/lemoq/kernels/_dequant_triton.py:313-463), y fp16 (y_is_f16) or fp32.
 * x fp16 contiguous, columns past K read as 0.  K <= padded_k <= 8192,
 * padded_k % group == 0, group % 16 == 0 (8-bit) or % 32 == 0 (4-bit; 32 for
 * MXFP4), 1 <= M <= 65535, qweight 16-byte aligned.  zero is required by the
 * asymmetric formats and ignored otherwise. */
int lemoq_gemv_q(const uint16_t* x, int64_t M, int64_t K, const void* qweight, int fmt,
                 const void* scale, const void* zero, int scale_is_f32, int64_t N,
                 int64_t padded_k, int64_t group, void* y, int y_is_f16, void* stream);

/* lemoq_gemv_q of the RMSNorm of x (the decoder layer's input norm before the
 * packed q|k|v projection, rms_norm_fused then dequant_gemm_fused,
 * src/lemoq/kernels/rmsnorm.py:102-163, _dequant_triton.py:155-293):
 * xn = fp16(fp16(x * rsqrt(mean(x^2) + eps)) * norm_w) with an fp32 mean over
 * K (lemoq_rmsnorm's rounding points; the fp32 sum of squares runs in another
 * order, so an element may differ from lemoq_rmsnorm's by one fp16 ulp), then
 * y = xn @ w^T as lemoq_gemv_q.  Rows that fill the kernel's 1 KB code chunks
 * exactly with K a multiple of 2048 (4-bit K 2048 / 4096 / 8192, 8-bit K 2048
 * / 4096 / 8192), x and norm_w 16-byte aligned, normalise once per block
 * (LDS); other rows in every wave.  With x_row_index (a device int64, M == 1)
 * the row is x[*x_row_index] of x_rows (the embedding gather of layer 0; an
 * index outside reads as a zero row); x_copy (nullable, needs the per-block
 * form, else LEMOQ_ERR_UNSUPPORTED) receives the raw row, written by block 0
 * (the residual stream).  norm_w (K) fp16; fp16 or E8M0 scales only
 * (scale_is_f32 returns LEMOQ_ERR_UNSUPPORTED); eps >= 0.  Used by the 4-bit
 * decode step. */
int lemoq_gemv_q_rmsnorm(const uint16_t* x, const int64_t* x_row_index, int64_t x_rows, int64_t M, int64_t K,
                         const uint16_t* norm_w, float eps, uint16_t* x_copy, const void* qweight, int fmt,
                         const void* scale, const void* zero, int scale_is_f32, int64_t N, int64_t padded_k,
                         int64_t group, void* y, int y_is_f16, void* stream);

/* lemoq_gemv_q with the fp16 residual add of the decoder layer after o_proj
 * (transformers OlmoeDecoderLayer.forward, the `residual + hidden_states` of
 * fp16 tensors): y (M, N) fp16 = fp16(fp16(x @ w^T) + residual), one rounding
 * of each.  residual (M, N) fp16 is y itself or apart from it (a partial
 * overlap returns LEMOQ_ERR_SHAPE).  Used by the 4-bit decode step. */
int lemoq_gemv_q_residual(const uint16_t* x, int64_t M, int64_t K, const void* qweight, int fmt,
                          const void* scale, const void* zero, int scale_is_f32, int64_t N,
                          int64_t padded_k, int64_t group, const uint16_t* residual, uint16_t* y,
                          void* stream);

/* lemoq_gemv_q on fp32 activations (the reference's dequant_gemm_fused takes
 * x fp16 or fp32, src/lemoq/kernels/_dequant_triton.py:252-253): the codes
 * become fp32 values and meet x in fp32 FMAs, fp32 accumulation.  Same
 * arguments and rules, x (M, K) fp32 contiguous. */
int lemoq_gemv_q_x32(const float* x, int64_t M, int64_t K, const void* qweight, int fmt,
                     const void* scale, const void* zero, int scale_is_f32, int64_t N,
                     int64_t padded_k, int64_t group, void* y, int y_is_f16, void* stream);

/* Dense weight of any LEMOQ_QFMT_* format: w[n][k] for k < k_out, computed
 * in fp32 and stored as fp32 (w_is_f32) or rounded once to fp16, rows ld_w
 * elements apart.  Replaces QuantLinear.dequantized_weight
 * (src/lemoq/quant/linear.py:365-395) and mxfp4.dequantize_packed
 * (src/lemoq/quant/mxfp4.py:105-122).  Same format rules as lemoq_gemv_q;
 * 1 <= k_out <= padded_k and ld_w >= k_out. */
int lemoq_dequant_q(const void* qweight, int fmt, const void* scale, const void* zero,
                    int scale_is_f32, int64_t N, int64_t padded_k, int64_t group, void* w,
                    int64_t ld_w, int64_t k_out, int w_is_f32, void* stream);

/* Per-token symmetric int8 fake quantisation of fp16 activations (x, y
 * (rows, D), may alias), the w8a8 scheme's QuantLinear._fake_quant_activation
 * (src/lemoq/quant/linear.py:398-414): fp32 absmax per row, s = absmax / 127
 * (1 when 0), q = clamp(rint(x / s), -128, 127), y = fp16(q * s). */
int lemoq_fake_quant_rows(const uint16_t* x, int64_t rows, int64_t D, uint16_t* y, void* stream);

/* ---------------------------------------------------------------------------
 * A7/A8/A9 — w8 symmetric dense GEMV (dequant in registers, fp32 accumulate).
 * Replaces dequant_gemm_fused(x, qweight, scale, None, group_size=g, bits=8,
 * symmetric=True, out_dtype=...) (src/lemoq/kernels/_dequant_triton.py:155-293,
 * kernel :313-463), the operator used by QuantLinear._fused_forward
 * (src/lemoq/quant/linear.py:446-469) and PackedQKV.project
 * (src/lemoq/kernels/packed_qkv.py:78-96).
 * x (M, K) fp16 contiguous; codes (N, padded_k) int8; scale (N, padded_k/group)
 * fp16; y (M, N) fp16 when y_is_f16 else fp32.  K <= padded_k <= 8192,
 * padded_k % 16 == 0, group % 16 == 0, padded_k % group == 0.
 * ------------------------------------------------------------------------- */
int lemoq_gemv_w8(const uint16_t* x, int64_t M, int64_t K,
                  const int8_t* codes, const uint16_t* scale, int64_t N,
                  int64_t padded_k, int64_t group, void* y, int y_is_f16,
                  void* stream);

/* Fused single-token form used by the decode step (no reference counterpart
 * as one call: it fuses rms_norm_fused (src/lemoq/kernels/rmsnorm.py:102-163)
 * into the GEMV prologue and the fp16 residual add of the HF decoder layer
 * (transformers OlmoeDecoderLayer.forward, call site
 * src/lemoq/kernels/attn_decode.py:1013-1016) into its epilogue).
 *   x_src:   the input row, or with x_row_index != NULL row *x_row_index of
 *            the (x_rows, K) table x_src (embedding gather; an index outside
 *            [0, x_rows) reads as a zero row).
 *   norm_w:  when non-NULL, x := fp16(fp16(x*rsqrt(mean(x^2)+eps)) * norm_w).
 *   x_copy:  when non-NULL, block 0 writes the raw (un-normed) input row here.
 *   residual: when non-NULL, y = fp16(fp16(acc) + residual) (may alias y).
 * K == padded_k here. */
int lemoq_gemv_w8_fused(const uint16_t* x_src, const int64_t* x_row_index,
                        int64_t x_rows, const uint16_t* norm_w, float eps,
                        uint16_t* x_copy,
                        const int8_t* codes, const uint16_t* scale, int64_t N,
                        int64_t K, int64_t group, const uint16_t* residual,
                        uint16_t* y, void* stream);

/* Fused final step of the decode graph (no single reference counterpart: it
 * joins the lm_head QuantLinear GEMV, src/lemoq/quant/linear.py:446-469, with
 * the greedy `logits.argmax()` of StaticCacheDecodeSession.replay,
 * benchmarks/cudagraph.py:759-762, moved onto the device).
 * logits (N) fp16 = W8 GEMV of x (optionally RMSNormed with norm_w); each
 * GEMV block writes its best (fp16 value, lowest row) to part_val/part_idx
 * (part_len >= lemoq_lm_head_argmax_parts(N)), then one block reduces them
 * (ties -> lowest row) and advances the step exactly like
 * lemoq_argmax_advance.  Two launches. */
int lemoq_lm_head_argmax_w8(const uint16_t* x, const uint16_t* norm_w, float eps,
                            const int8_t* codes, const uint16_t* scale, int64_t N, int64_t K,
                            int64_t group, uint16_t* logits, float* part_val,
                            int32_t* part_idx, int64_t part_len, int64_t* token, int64_t* pos,
                            int32_t* filled, const int64_t* prompt, int64_t prompt_len,
                            int64_t* history, int64_t history_len, void* stream);
/* The same two launches with the lm_head arithmetic of the multi-token
 * QuantLinear arm (src/lemoq/quant/linear.py:420-434, :365-395): each weight
 * rounded to fp16(code * scale) before fp32 dot products, as the prefill's
 * F.linear over the dequantised lm_head computes the last position's logits
 * (the prefill forward, benchmarks/cudagraph.py:578-599), followed by the
 * greedy pick of the seed token.  Arguments and errors as
 * lemoq_lm_head_argmax_w8. */
int lemoq_lm_head_argmax_w8_dq(const uint16_t* x, const uint16_t* norm_w, float eps,
                               const int8_t* codes, const uint16_t* scale, int64_t N, int64_t K,
                               int64_t group, uint16_t* logits, float* part_val,
                               int32_t* part_idx, int64_t part_len, int64_t* token, int64_t* pos,
                               int32_t* filled, const int64_t* prompt, int64_t prompt_len,
                               int64_t* history, int64_t history_len, void* stream);
/* The same two launches over an fp16 lm_head (the w4a16 cell keeps lm_head
 * in fp16, benchmarks/runner.py:399-401 and src/lemoq/quant/linear.py:646-647,
 * so its logits are a plain F.linear; the greedy pick of
 * benchmarks/cudagraph.py:759-762).  weight (N, K)
 * fp16 row-major; logits = fp16(rmsnorm(x, norm_w) . W[n]) with fp32
 * accumulation, bit-identical to lemoq_router_logits over the same rows;
 * part_len >= lemoq_lm_head_argmax_parts(N).  K % 16 == 0, K <= 8192;
 * 16-byte aligned x, weight and norm_w (else LEMOQ_ERR_ALIGN). */
int lemoq_lm_head_argmax_f16(const uint16_t* x, const uint16_t* norm_w, float eps,
                             const uint16_t* weight, int64_t N, int64_t K, uint16_t* logits,
                             float* part_val, int32_t* part_idx, int64_t part_len, int64_t* token,
                             int64_t* pos, int32_t* filled, const int64_t* prompt,
                             int64_t prompt_len, int64_t* history, int64_t history_len,
                             void* stream);
/* Number of argmax partials lemoq_lm_head_argmax_w8 writes for N rows. */
int64_t lemoq_lm_head_argmax_parts(int64_t N);

/* ---------------------------------------------------------------------------
 * A4 — grouped MoE gate/up + SiLU, w8.
 * Replaces _gate_up_act_kernel_q (src/lemoq/kernels/_grouped_triton.py:249-332)
 * as launched by grouped_moe_forward_quant
 * (src/lemoq/kernels/moe_grouped_quant.py:473-515).
 * x (H,) fp16; codes (E, 2F, H) int8 (gate rows [0,F), up rows [F,2F));
 * scale (E, 2F, H/group) fp16; ids (top_k,) int64 device;
 * act (top_k, F) fp16 = fp16(silu(gate) * up), fp32 accumulation.
 * An id outside [0, E) yields a zero row (no out-of-bounds read).
 * ------------------------------------------------------------------------- */
int lemoq_moe_gate_up_w8(const uint16_t* x, const int8_t* codes,
                         const uint16_t* scale, const int64_t* ids,
                         int64_t top_k, int64_t num_experts, int64_t ffn,
                         int64_t hidden, int64_t group, uint16_t* act,
                         void* stream);

/* Routed form used by the decode step: takes the router's fp16 logits (E)
 * instead of ids.  Every wave runs the routing of lemoq_route_topk (fp32
 * softmax, top_k with ties -> lowest index, optional renormalisation) and
 * streams the expert of its slot; the selected ids (int64) and fp16 weights
 * (the `.to(x.dtype)` of moe_static._route, src/lemoq/kernels/moe_static.py:
 * 276-283) are stored to top_i/top_w for the down kernel.  E <= 256,
 * top_k <= 64. */
int lemoq_moe_gate_up_w8_routed(const uint16_t* x, const int8_t* codes,
                                const uint16_t* scale, const uint16_t* router_logits,
                                int64_t top_k, int norm_topk_prob, int64_t num_experts,
                                int64_t ffn, int64_t hidden, int64_t group, uint16_t* act,
                                int64_t* top_i, uint16_t* top_w, void* stream);

/* A5 — grouped MoE down projection x routing weight, summed over the top_k
 * slots in a fixed order, fp32 accumulation, fp16 output.  Replaces
 * _down_sum_kernel_q + _out_reduce_kernel
 * (src/lemoq/kernels/_grouped_triton.py:335-398, :197-211) as launched at
 * src/lemoq/kernels/moe_grouped_quant.py:517-558.
 * act (top_k, F) fp16; codes (E, H, F) int8; scale (E, H, F/group) fp16;
 * ids (top_k,) int64; top_w (top_k,) fp16; out (H,) fp16.
 * residual (nullable, may alias out): out = fp16(fp16(sum) + residual). */
int lemoq_moe_down_w8(const uint16_t* act, const int8_t* codes,
                      const uint16_t* scale, const int64_t* ids,
                      const uint16_t* top_w, int64_t top_k, int64_t num_experts,
                      int64_t hidden, int64_t ffn, int64_t group,
                      const uint16_t* residual, uint16_t* out, void* stream);

/* A4/A5 on 4-bit symmetric experts (the BITS=4 branch of the same kernels,
 * src/lemoq/kernels/_grouped_triton.py:235-398, and of
 * quantize_fused_experts(bits=4), src/lemoq/kernels/moe_grouped_quant.py:191-244).
 * codes are int4 (-8..7) packed two per byte, the even column in the low
 * nibble: gate/up (E, 2F, H/2), down (E, H, F/2); scales fp16 per group of
 * `group` codes.  Arguments, outputs and numerics as the 8-bit entry points;
 * hidden and ffn <= 8192, multiples of 32 and of group, group % 32 == 0. */
int lemoq_moe_gate_up_w4(const uint16_t* x, const uint8_t* codes, const uint16_t* scale,
                         const int64_t* ids, int64_t top_k, int64_t num_experts, int64_t ffn,
                         int64_t hidden, int64_t group, uint16_t* act, void* stream);
/* Routed form of lemoq_moe_gate_up_w4, as lemoq_moe_gate_up_w8_routed: the
 * router's fp16 logits (E) in place of ids, routing in every block (ties ->
 * lowest index), the selected ids and fp16 weights stored to top_i / top_w.
 * E <= 256, top_k <= 64.  Used by the 4-bit decode step. */
int lemoq_moe_gate_up_w4_routed(const uint16_t* x, const uint8_t* codes, const uint16_t* scale,
                                const uint16_t* router_logits, int64_t top_k, int norm_topk_prob,
                                int64_t num_experts, int64_t ffn, int64_t hidden, int64_t group,
                                uint16_t* act, int64_t* top_i, uint16_t* top_w, void* stream);
int lemoq_moe_down_w4(const uint16_t* act, const uint8_t* codes, const uint16_t* scale,
                      const int64_t* ids, const uint16_t* top_w, int64_t top_k,
                      int64_t num_experts, int64_t hidden, int64_t ffn, int64_t group,
                      const uint16_t* residual, uint16_t* out, void* stream);

/* ---------------------------------------------------------------------------
 * A14/A15 — split-KV decode attention (flash-decoding), batch 1, q_len 1.
 * Partials: m, l (heads, num_splits) fp32 and acc (heads, num_splits, D) fp32;
 * split s of head h covers [s*c, min((s+1)*c, filled)) with
 * c = ceil(filled/num_splits), filled read from the device int32 *filled.
 * Scores use exp2 with qk_scale = scale*log2(e); an empty split writes
 * (m=-inf, l=0, acc=0).  D in {64, 128, 256}.
 *
 * fp16 K/V: replaces _attn_split_kernel (src/lemoq/kernels/_attn_triton.py:46-99)
 * launched by attn_decode_forward (src/lemoq/kernels/attn_decode.py:496-624).
 * q (heads, D) fp16; k, v: head h, token t at k + h*head_stride + t*D. */
int lemoq_attn_split_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         int64_t head_stride, const int32_t* filled,
                         int64_t heads, int64_t head_dim, int64_t num_splits,
                         float qk_scale, float* m, float* l, float* acc,
                         void* stream);

/* KV-INT8: replaces _attn_split_kernel_int8 (src/lemoq/kernels/_attn_triton.py:102-165)
 * launched by attn_decode_forward_int8 (src/lemoq/kernels/attn_decode.py:627-730).
 * score_t = ((q . c_t) * qk_scale) * ks_t;  acc += sum_t (p_t * vs_t) * cv_t;
 * l = sum_t p_t (the V scale is not in l).  Codes: kc + h*head_stride + t*D;
 * scales: ks + h*s_len + t. */
int lemoq_attn_split_i8(const uint16_t* q, const int8_t* kc, const uint16_t* ks,
                        const int8_t* vc, const uint16_t* vs, int64_t head_stride,
                        int64_t s_len, const int32_t* filled, int64_t heads,
                        int64_t head_dim, int64_t num_splits, float qk_scale,
                        float* m, float* l, float* acc, void* stream);

/* LSE merge, fixed split order: out = sum_j acc_j 2^(m_j-M) / sum_j l_j 2^(m_j-M),
 * M = max_j m_j (0 when every split is empty, giving out = 0).  Replaces
 * _attn_combine_kernel (src/lemoq/kernels/_attn_triton.py:168-206).
 * out (heads, D) fp16. */
int lemoq_attn_merge(const float* m, const float* l, const float* acc,
                     int64_t heads, int64_t num_splits, int64_t head_dim,
                     uint16_t* out, void* stream);

/* LSE merge fused into the w8 o_proj GEMV, split over groups of 4 heads (no
 * reference counterpart as one call: it joins _attn_combine_kernel
 * (src/lemoq/kernels/_attn_triton.py:168-206) and the o_proj QuantLinear of
 * the attention forward (src/lemoq/kernels/attn_decode.py:1015, fused GEMV
 * arm src/lemoq/quant/linear.py:431-434)).  Block column g merges heads
 * 4g..4g+3 with the arithmetic of lemoq_attn_merge (bit-identical fp16
 * attention output) and writes
 *   part[g][n] = sum over input features k in [512g, 512g+512) of
 *                scale[n][k/group] * code[n][k] * attn[k]   (fp32),
 * so that o = fp16(sum_g part[g]) is the o_proj output.  head_dim == 128,
 * heads % 4 == 0, num_splits <= 64, N % 32 == 0, group % 16 == 0.
 *   m, l (heads, num_splits); acc (heads, num_splits, 128) fp32;
 *   codes (N, heads*128) int8; scale (N, heads*128/group) fp16;
 *   part (heads/4, N) fp32. */
int lemoq_attn_merge_o_proj_w8(const float* m, const float* l, const float* acc,
                               int64_t heads, int64_t num_splits, int64_t head_dim,
                               const int8_t* codes, const uint16_t* scale, int64_t N,
                               int64_t group, float* part, void* stream);
/* The same on 4-bit symmetric codes (the w4a16 cell's o_proj, the 4-bit
 * branch of dequant_gemm_fused, src/lemoq/kernels/_dequant_triton.py:155-293):
 * codes (N, heads*128/2) packed two per byte, the even column in the low
 * nibble; group % 32 == 0.  Used by the 4-bit decode step. */
int lemoq_attn_merge_o_proj_w4(const float* m, const float* l, const float* acc,
                               int64_t heads, int64_t num_splits, int64_t head_dim,
                               const uint8_t* codes, const uint16_t* scale, int64_t N,
                               int64_t group, float* part, void* stream);

/* ---------------------------------------------------------------------------
 * A10 — RMSNorm, HF rounding points: y = fp16(fp16(x*rsqrt(mean(x^2)+eps)) * w).
 * Replaces rms_norm_fused (src/lemoq/kernels/rmsnorm.py:102-163, kernel
 * :173-202).  x, y (rows, hidden) fp16 contiguous; w (hidden,) fp16;
 * hidden <= 8192.  Rows with hidden % 8 == 0 and x, w, y 16-byte aligned are
 * read in 16-byte chunks; other rows one element per thread, which sums the
 * squares in another fp32 order, so the two can differ by an fp16 ulp on the
 * same row (the rounding points are the same).
 * ------------------------------------------------------------------------- */
int lemoq_rmsnorm(const uint16_t* x, int64_t rows, int64_t hidden,
                  const uint16_t* w, float eps, uint16_t* y, void* stream);

/* A11 — rotary embedding on one (1, heads, 1, D) tensor, strided:
 * out = x*cos + rotate_half(x)*sin in fp32, rounded to fp16.  Replaces
 * _rope_one_kernel (src/lemoq/kernels/rope.py:86-123) as launched by
 * apply_rotary_pos_emb_fused (src/lemoq/kernels/rope.py:154-203).
 * Element (h, d) of x at x + h*x_sh + d*x_sd; cos/sin element d at
 * cos + d*cs_sd; out element at out + h*o_sh + d*o_sd.  D even, D <= 1024. */
int lemoq_rope(const uint16_t* x, int64_t x_sh, int64_t x_sd, int64_t heads,
               int64_t head_dim, const uint16_t* cos, const uint16_t* sin,
               int64_t cs_sd, uint16_t* out, int64_t o_sh, int64_t o_sd,
               void* stream);

/* ---------------------------------------------------------------------------
 * A12 — bitwise copy of the new k/v rows (heads, D) fp16 to slot *pos of the
 * fp16 cache.  Replaces _kv_direct_write_kernel / kv_direct_write
 * (src/lemoq/kernels/kv_direct.py:78-137; contract kv_write.py:26-50).
 * Source head h at k + h*src_head_stride; destination at
 * k_cache + h*dst_head_stride + (*pos)*D.  pos is a device int64.
 * ------------------------------------------------------------------------- */
int lemoq_kv_write_f16(const uint16_t* k, const uint16_t* v,
                       int64_t src_head_stride, uint16_t* k_cache,
                       uint16_t* v_cache, int64_t dst_head_stride,
                       const int64_t* pos, int64_t heads, int64_t head_dim,
                       void* stream);

/* A13 — KV direct-write quantisation.  Per (head) row of the new k and v:
 * s = fp32(amax)/127 (1.0 when amax == 0), code = round-half-even(x/s)
 * clamped to [-127, 127], scale stored as fp16(s).  Codes of head h go to
 * kc + h*code_head_stride + slot*D, the scale to ks + h*s_len + slot, with
 * slot = *pos (device int64) or 0 when pos is NULL.  Replaces
 * _kv_int8_cache_write_kernel / kv_int8_cache_write
 * (src/lemoq/kernels/kv_int8.py:182-257) and, with pos == NULL,
 * code_head_stride == D and s_len == 1, kv_int8_write (:276-355). */
int lemoq_kv_write_i8(const uint16_t* k, const uint16_t* v, int64_t heads,
                      int64_t head_dim, int8_t* kc, uint16_t* ks, int8_t* vc,
                      uint16_t* vs, int64_t code_head_stride, int64_t s_len,
                      const int64_t* pos, void* stream);

/* Bulk per-token quantisation of `rows` contiguous rows of D fp16 (same
 * arithmetic as lemoq_kv_write_i8).  Replaces kv_int8_bulk_quantize
 * (src/lemoq/kernels/kv_int8.py:127-163). */
int lemoq_kv_quantize_rows(const uint16_t* x, int64_t rows, int64_t head_dim,
                           int8_t* codes, uint16_t* scales, void* stream);

/* ---------------------------------------------------------------------------
 * A3 — routing: fp32 softmax over E logits, top_k by value (ties -> lowest
 * index), optional renormalisation over the selected k.  Replaces
 * _routing_softmax_topk_kernel / routing_softmax_topk
 * (src/lemoq/kernels/_routing_triton.py:43-130).
 * logits (T, E) with row stride `row_stride` elements, fp16 when
 * logits_is_f16 else fp32; top_w (T, top_k) fp32; top_i (T, top_k) int64.
 * E <= 1024, top_k <= E.
 * ------------------------------------------------------------------------- */
int lemoq_route_topk(const void* logits, int logits_is_f16, int64_t T, int64_t E,
                     int64_t row_stride, int64_t top_k, int norm_topk_prob,
                     float* top_w, int64_t* top_i, void* stream);

/* lemoq_route_topk on the logits lemoq_gemm_f16_splitk would produce from
 * `partials` ((splits, T, E) fp32, its workspace): each logit is the fp16
 * rounding of the partials summed in range order from 0, as that entry's
 * second launch computes it, so the routing is identical while the sum and
 * the routing share one launch (prefill's router, the same F.linear and
 * routing_softmax_topk as lemoq_route_topk).  1 <= splits <= 64. */
int lemoq_route_topk_splitk(const float* partials, int64_t splits, int64_t T, int64_t E,
                            int64_t top_k, int norm_topk_prob, float* top_w, int64_t* top_i,
                            void* stream);

/* Router logits of one token: xn = rmsnorm(h, norm_w) (xn_out, nullable),
 * logits_out (E) = fp16(xn @ router_w^T), fp32 accumulation (the F.linear of
 * moe_static._route, src/lemoq/kernels/moe_static.py:267).  One wave per
 * expert row over ceil(E/4) blocks; hidden % 16 == 0, 16-byte aligned
 * pointers. */
int lemoq_router_logits(const uint16_t* h, const uint16_t* norm_w, float eps, int64_t hidden,
                        const uint16_t* router_w, int64_t E, uint16_t* xn_out,
                        uint16_t* logits_out, void* stream);

/* Router logits after the o_proj partials of lemoq_attn_merge_o_proj_w8 (no
 * reference counterpart as one call: the fp16 residual add after o_proj
 * (transformers OlmoeDecoderLayer.forward), post_attention_layernorm
 * (rms_norm_fused, src/lemoq/kernels/rmsnorm.py:102-163) and the router
 * F.linear of moe_static._route (src/lemoq/kernels/moe_static.py:267)):
 *   o = fp16(sum_g part[g]) (g ascending), h_out = fp16(o + h),
 *   xn = rmsnorm(h_out, norm_w) (xn_out, nullable; block 0 writes it and
 *   h_out), logits (E) = fp16(xn @ router_w^T) with fp32 accumulation.
 * hidden in {2048, 4096}, n_part in {1, 2, 4, 8}; part (n_part, hidden) fp32;
 * 16-byte aligned pointers; h_out must not overlap h or part. */
int lemoq_router_logits_resid(const float* part, int64_t n_part, const uint16_t* h,
                              const uint16_t* norm_w, float eps, int64_t hidden,
                              const uint16_t* router_w, int64_t E, uint16_t* h_out,
                              uint16_t* xn_out, uint16_t* logits, void* stream);


/* Router of one token, fused: xn = rmsnorm(h, norm_w) (written to xn_out),
 * logits = fp16(xn @ router_w^T) with fp32 accumulation (the F.linear of
 * moe_static._route, src/lemoq/kernels/moe_static.py:262-283), then the
 * routing above; top_w_f16 = fp16(top_w) (the `.to(x.dtype)` of _route).
 * router_w (E, hidden) fp16.  norm_w may be NULL (no norm: xn = h).
 * logits_out, top_w_f32 and top_w_f16 may be NULL.  One 1024-thread block
 * (the 64 x 2048 router is 256 KB; one wave per row, then one wave routes). */
int lemoq_router_topk_fused(const uint16_t* h, const uint16_t* norm_w, float eps,
                            int64_t hidden, const uint16_t* router_w, int64_t E,
                            int64_t top_k, int norm_topk_prob, uint16_t* xn_out,
                            uint16_t* logits_out, float* top_w_f32,
                            uint16_t* top_w_f16, int64_t* top_i, void* stream);

/* ---------------------------------------------------------------------------
 * A16 — per-layer attention prologue of the decode step, fused: from the
 * packed q|k|v row (3*heads*D fp16) computes q_norm and k_norm (RMSNorm over
 * heads*D, HF rounding), RoPE with the cos/sin row (*pos) of the tables
 * cos_tab/sin_tab (max_pos, D) fp16, writes q_out (heads, D) fp16, and writes
 * the new k and v rows KV-INT8-quantised to slot *pos (same arithmetic as
 * lemoq_kv_write_i8).  k_f16/v_f16 (nullable): also copy the fp16 rows into an
 * fp16 cache at h*f16_head_stride + (*pos)*D.  k_rot_out (nullable): the
 * fp16 rotated k row, for tests.  clip_qkv: HF OLMoE's clip_qkv, applied as
 * the reference applies it (src/lemoq/kernels/attn_decode.py:903-907, after
 * q_norm/k_norm, before RoPE, and to v): values beyond +-clip_qkv become
 * +-fp16(clip_qkv), NaN stays; +INFINITY disables it; a negative or NaN bound
 * is rejected.  Replaces the sequence at src/lemoq/kernels/attn_decode.py:882-987.
 * ------------------------------------------------------------------------- */
int lemoq_qk_norm_rope_kv_i8(const uint16_t* qkv, int64_t heads, int64_t head_dim,
                             const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                             float eps, const uint16_t* cos_tab,
                             const uint16_t* sin_tab, const int64_t* pos,
                             uint16_t* q_out, int8_t* kc, uint16_t* ks, int8_t* vc,
                             uint16_t* vs, int64_t code_head_stride, int64_t s_len,
                             uint16_t* k_f16, uint16_t* v_f16,
                             int64_t f16_head_stride, uint16_t* k_rot_out,
                             float clip_qkv, void* stream);

/* A16 fused (no reference counterpart as one call: it joins the q_norm/k_norm,
 * RoPE, KV-INT8 write and split-KV int8 attention sequence of
 * src/lemoq/kernels/attn_decode.py:882-1000 for one decode token).  Grid
 * (num_splits, heads): split s of head h covers [s*c, min((s+1)*c, n)) with
 * n = *pos + 1, c = ceil(n/num_splits).  From the packed q|k|v row, q and the
 * new k are RMS-normed over heads*D and rotated at *pos; the block holding
 * *pos quantises the new k and v to KV-INT8 and writes them to slot *pos
 * (same arithmetic, clip_qkv included, and bytes as lemoq_qk_norm_rope_kv_i8).  Writes the
 * partials m, l (heads, num_splits) and acc (heads, num_splits, D) of
 * lemoq_attn_split_i8 over tokens [0, *pos]; merge them with
 * lemoq_attn_merge.  D in {64, 128, 256}. */
int lemoq_attn_split_fused_i8(const uint16_t* qkv, int64_t heads, int64_t head_dim,
                              const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps,
                              const uint16_t* cos_tab, const uint16_t* sin_tab,
                              const int64_t* pos, int8_t* kc, uint16_t* ks, int8_t* vc,
                              uint16_t* vs, int64_t code_head_stride, int64_t s_len,
                              int64_t num_splits, float qk_scale, float* m, float* l, float* acc,
                              float clip_qkv, void* stream);

/* A16 fused over the fp16 cache (KV-INT8 off): the q_norm/k_norm, RoPE,
 * kv_direct_write and fp16 split-KV attention sequence of
 * src/lemoq/kernels/attn_decode.py:882-948,999-1008 (kv_direct.py:110-137,
 * _attn_triton.py:30-99) for one decode token.  As lemoq_attn_split_fused_i8,
 * except that the block holding *pos writes the rotated k row and the v row
 * as fp16 to slot *pos of kc / vc ((heads, head_stride) fp16, head_stride >=
 * s_len*D elements, 16-byte aligned rows) -- the bits lemoq_qk_norm_rope_kv_i8
 * gives for them -- and the partials are those of lemoq_attn_split_f16 over
 * tokens [0, *pos] (the same arithmetic; the token order within a split may
 * differ, so the sums agree to fp32 rounding). */
int lemoq_attn_split_fused_f16(const uint16_t* qkv, int64_t heads, int64_t head_dim,
                               const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps,
                               const uint16_t* cos_tab, const uint16_t* sin_tab,
                               const int64_t* pos, uint16_t* kc, uint16_t* vc, int64_t head_stride,
                               int64_t s_len, int64_t num_splits, float qk_scale, float* m, float* l,
                               float* acc, float clip_qkv, void* stream);

/* ---------------------------------------------------------------------------
 * A17 — greedy selection and step advance on the device (replaces the host
 * `logits.argmax().item()` of StaticCacheDecodeSession.replay,
 * benchmarks/cudagraph.py:751-766, and the per-step fills of
 * _set_step_inputs, :655-678).  next = argmax(logits[0:n]) (first index on
 * ties), or prompt[*pos + 1] while *pos + 1 < prompt_len; then
 * *token = next, history[*pos + 1] = next (when *pos + 1 < history_len),
 * *pos += 1, *filled = *pos + 1.  0 < n < 2^31.
 * ------------------------------------------------------------------------- */
int lemoq_argmax_advance(const uint16_t* logits, int64_t n, int64_t* token,
                         int64_t* pos, int32_t* filled, const int64_t* prompt,
                         int64_t prompt_len, int64_t* history, int64_t history_len,
                         void* stream);

/* ---------------------------------------------------------------------------
 * A17/A18 — one whole OLMoE decode step (embedding -> 16 x [attention, MoE]
 * -> final norm -> lm_head -> greedy advance) enqueued on `stream`; the
 * caller captures it into a hipGraph.  Replaces the captured
 * model(token, ...) forward of StaticCacheDecodeSession.capture
 * (benchmarks/cudagraph.py:680-737) for the canonical w8a16 + W8 lm_head +
 * KV-INT8 cell, or, with kv_fp16 set, the same cell with KV-INT8 off (the
 * fp16 StaticCache written by kv_direct_write and read by the fp16 split-KV
 * attention, src/lemoq/kernels/attn_decode.py:930-948,999-1008), or, with
 * weight_bits 4 and lm_f16, the w4a16 cell (benchmarks/runner.py:393-412,
 * 451-482).  All buffers are caller-owned; see LemoqOlmoeStep.
 * ------------------------------------------------------------------------- */
typedef struct LemoqOlmoeLayer {
  const uint16_t* ln_in;     /* (H)                */
  const uint16_t* ln_post;   /* (H)                */
  const uint16_t* q_norm;    /* (heads*D)          */
  const uint16_t* k_norm;    /* (heads*D)          */
  const int8_t* qkv_codes;   /* (3*heads*D, H); the code arrays are packed 4-bit at weight_bits 4 */
  const uint16_t* qkv_scale; /* (3*heads*D, H/g)   */
  const int8_t* o_codes;     /* (H, heads*D)       */
  const uint16_t* o_scale;   /* (H, heads*D/g)     */
  const uint16_t* router;    /* (E, H) fp16        */
  const int8_t* gu_codes;    /* (E, 2F, H)         */
  const uint16_t* gu_scale;  /* (E, 2F, H/g)       */
  const int8_t* dn_codes;    /* (E, H, F)          */
  const uint16_t* dn_scale;  /* (E, H, F/g)        */
  int8_t* kc;                /* (heads, S, D) int8; fp16 rows when kv_fp16 */
  uint16_t* ks;              /* (heads, S); unused (may be NULL) when kv_fp16 */
  int8_t* vc;                /* (heads, S, D) int8; fp16 rows when kv_fp16 */
  uint16_t* vs;              /* (heads, S); unused (may be NULL) when kv_fp16 */
} LemoqOlmoeLayer;

typedef struct LemoqOlmoeStep {
  /* shapes */
  int64_t hidden, heads, head_dim, ffn, num_experts, top_k, vocab, group;
  int64_t num_layers, max_seq, num_splits, norm_topk_prob;
  float eps, qk_scale;
  float clip_qkv;                /* HF clip_qkv (+INFINITY: none); see lemoq_qk_norm_rope_kv_i8 */
  /* weights */
  const LemoqOlmoeLayer* layers; /* host array of num_layers entries */
  const uint16_t* embed;         /* (vocab, H) fp16 */
  const uint16_t* final_norm;    /* (H) */
  const int8_t* lm_codes;        /* (vocab, H) */
  const uint16_t* lm_scale;      /* (vocab, H/g) */
  const uint16_t* cos_tab;       /* (max_seq, D) fp16 */
  const uint16_t* sin_tab;       /* (max_seq, D) fp16 */
  /* device scalars and per-step buffers */
  int64_t* token;                /* (1) current token id */
  int64_t* pos;                  /* (1) position of `token` */
  int32_t* filled;               /* (1) == *pos + 1 during the step */
  const int64_t* prompt;         /* (prompt_len) */
  int64_t prompt_len;
  int64_t* history;              /* (history_len) token at each position */
  int64_t history_len;
  uint16_t* h;                   /* (H) residual stream */
  uint16_t* xn;                  /* (H) normed input of the MoE */
  uint16_t* qkv;                 /* (3*heads*D) */
  uint16_t* q_rot;               /* (heads*D) */
  uint16_t* attn;                /* (heads*D) */
  float* part_m;                 /* (heads*num_splits) */
  float* part_l;                 /* (heads*num_splits) */
  float* part_acc;               /* (heads*num_splits*D) */
  uint16_t* router_logits;       /* (E) */
  uint16_t* top_w;               /* (top_k) fp16 */
  int64_t* top_i;                /* (top_k) */
  uint16_t* act;                 /* (top_k, F) */
  uint16_t* logits;              /* (vocab) fp16 */
  float* am_val;                 /* (am_len) argmax partials */
  int32_t* am_idx;               /* (am_len) */
  int64_t am_len;                /* >= lemoq_lm_head_argmax_parts(vocab) */
  /* Fused attention-output path (merge + o_proj, then residual + norm +
   * router in the next launch), used when both are non-NULL and the shapes
   * allow it (head_dim 128, heads % 4 == 0, num_splits <= 64, hidden 2048
   * or 4096, heads*128/512 partial rows in {1, 2, 4, 8}); otherwise the step
   * runs lemoq_attn_merge, the o_proj GEMV and lemoq_router_logits. */
  float* o_part;                 /* (heads*D/512, H) o_proj partial sums */
  uint16_t* h_mid;               /* (H) residual after attention */
  /* Cache kind: 0 = KV-INT8 (kc/vc int8 codes, ks/vs fp16 scales), 1 = fp16
   * rows (kc/vc point to (heads, S, D) fp16; lemoq_attn_split_fused_f16). */
  int64_t kv_fp16;
  /* Attention and expert weight bits: 8 (the layer's codes as declared
   * above) or 4 (the reference's w4a16 cell: 4-bit symmetric codes packed two
   * per byte, the even column in the low nibble, so qkv_codes (3*heads*D,
   * H/2), o_codes (H, heads*D/2), gu_codes (E, 2F, H/2), dn_codes (E, H, F/2);
   * scales as above; group % 32 == 0).  A 4-bit step runs 6 launches per
   * layer on the fused attention-output path (the shape rule below):
   * lemoq_gemv_q_rmsnorm (input norm + q|k|v; layer 0 gathers the embedding
   * row and stores it to h), the fused attention,
   * lemoq_attn_merge_o_proj_w4, lemoq_router_logits_resid,
   * lemoq_moe_gate_up_w4_routed, lemoq_moe_down_w4 (+ residual); otherwise 7,
   * with lemoq_attn_merge, lemoq_gemv_q_residual (o_proj + residual into h)
   * and lemoq_router_logits in place of the middle two.  (When the q|k|v
   * GEMV's rows do not take its per-block norm, layer 0 first gathers the
   * embedding row into h with lemoq_gather_rows.) */
  int64_t weight_bits;
  /* fp16 lm_head (vocab, H), or NULL for the W8 lm_head of lm_codes /
   * lm_scale.  With it the step ends with lemoq_lm_head_argmax_f16 (final
   * norm + fp16 GEMV writing the argmax partials to am_val / am_idx, then
   * the pick); the reference keeps the lm_head in fp16 in every cell but
   * w8a16 with its lm_head switch on. */
  const uint16_t* lm_f16;
} LemoqOlmoeStep;

int lemoq_olmoe_decode_step(const LemoqOlmoeStep* step, void* stream);

/* ---------------------------------------------------------------------------
 * Prefill (several tokens per call) — batched GEMMs on the matrix cores.
 *
 * w8 linear over M rows with the numerics of the reference's multi-token
 * QuantLinear arm ("separate": dequantised fp16 weight, then F.linear;
 * src/lemoq/quant/linear.py:365-395,471-480, chosen for every input with more
 * than one token, :431-434): w = fp16(code * scale), fp32 accumulation,
 * y = fp16(x @ w^T); with residual != NULL, y = fp16(y + residual) (torch's
 * fp16 add).  x row m is row x_rows[m] of x when x_rows != NULL.
 *   x (rows, x_ld) fp16; codes (N, K) int8; scale (N, K/group) fp16;
 *   y (M, y_ld) fp16; residual (M, residual_ld) fp16 (may alias y).
 *   K % 64 == 0, group % 64 == 0, K % group == 0, x_ld % 8 == 0, x and codes
 *   16-byte aligned.
 * ------------------------------------------------------------------------- */
int lemoq_gemm_w8(const uint16_t* x, int64_t M, int64_t K, int64_t x_ld, const int32_t* x_rows,
                  const int8_t* codes, const uint16_t* scale, int64_t N, int64_t group,
                  uint16_t* y, int64_t y_ld, const uint16_t* residual, int64_t residual_ld,
                  void* stream);

/* fp16 linear over M rows, y = fp16(x @ w^T) with fp32 accumulation: the
 * router's F.linear for several tokens (src/lemoq/kernels/moe_static.py:267).
 *   w (N, K) fp16; same shape rules as lemoq_gemm_w8. */
int lemoq_gemm_f16(const uint16_t* x, int64_t M, int64_t K, int64_t x_ld, const uint16_t* w,
                   int64_t N, uint16_t* y, int64_t y_ld, void* stream);

/* lemoq_gemm_f16 for narrow outputs (the 64-expert router): K is cut into
 * `splits` ranges (K % (64 * splits) == 0, splits <= 64), each range's fp32
 * partial goes to workspace ((splits, M, N) fp32, 16-byte aligned, caller-
 * owned), and a second launch sums the partials in range order and rounds
 * once to fp16.  splits == 1 is lemoq_gemm_f16 (workspace unused).  With
 * splits > 1, y == NULL leaves the partials in workspace and skips the sum
 * (lemoq_route_topk_splitk finishes them). */
int lemoq_gemm_f16_splitk(const uint16_t* x, int64_t M, int64_t K, int64_t x_ld, const uint16_t* w,
                          int64_t N, uint16_t* y, int64_t y_ld, int64_t splits, float* workspace,
                          void* stream);

/* lemoq_gemm_f16_splitk for callers that cannot allocate (code under hipGraph
 * capture, serving loops, harnesses that forbid hipMalloc): no reference
 * counterpart.  The split partials go to a fixed device array of
 * LEMOQ_SPLITK_SCRATCH_FLOATS floats (16 MiB) that the library holds on each
 * device it runs on until the process ends; the call itself allocates
 * nothing.  Requires y (the partials cannot be left for the caller) and
 * splits * M * N <= LEMOQ_SPLITK_SCRATCH_FLOATS when splits > 1, else returns
 * LEMOQ_ERR_CAPACITY before launching.  All calls on one device share the
 * array: calls that overlap in time on one device (other streams, other
 * threads) race and must be serialised by the caller.  Same results as
 * lemoq_gemm_f16_splitk bit for bit. */
#define LEMOQ_SPLITK_SCRATCH_FLOATS (4 << 20)
int lemoq_gemm_f16_splitk_noalloc(const uint16_t* x, int64_t M, int64_t K, int64_t x_ld, const uint16_t* w,
                                  int64_t N, uint16_t* y, int64_t y_ld, int64_t splits, void* stream);

/* Embedding lookup of several tokens (HF embed_tokens on the prompt):
 * dst[r] = src[ids[r]] for r < rows, a zero row for an id outside
 * [0, n_rows).  src (n_rows, H) fp16, dst (rows, H); H % 8 == 0, 16-byte
 * aligned. */
int lemoq_gather_rows(const uint16_t* src, int64_t n_rows, int64_t H, const int64_t* ids, int64_t rows,
                      uint16_t* dst, void* stream);

/* Attention prologue of several prompt rows: lemoq_qk_norm_rope_kv_i8 per row
 * r of qkv (rows, 3*heads*D) at position pos0 + r, with the RoPE rounding of
 * HF's apply_rotary_pos_emb (fp16(fp16(x*cos) + fp16(rotate_half(x)*sin))),
 * which the reference's multi-token path uses (the fused RoPE guard takes
 * q_len == 1 only, src/lemoq/kernels/rope.py:140-177).  q_out (rows, heads,
 * D); KV-INT8 rows into slots pos0 .. pos0+rows-1 (the values
 * kv_int8_bulk_quantize, src/lemoq/kernels/kv_int8.py:127-162, gives for the
 * fp16 cache rows); k_f16/v_f16 (nullable) fp16 copies at
 * h*f16_head_stride + pos*D for the prefill attention.  With kc, ks, vc and
 * vs all NULL no KV-INT8 rows are written and k_f16/v_f16 (then required)
 * are the fp16 cache itself (KV-INT8 off).  pos0 + rows <= s_len;
 * cos_tab/sin_tab hold s_len rows.  clip_qkv as for lemoq_qk_norm_rope_kv_i8. */
int lemoq_qk_norm_rope_kv_i8_rows(const uint16_t* qkv, int64_t rows, int64_t heads,
                                  int64_t head_dim, const uint16_t* q_norm_w,
                                  const uint16_t* k_norm_w, float eps, const uint16_t* cos_tab,
                                  const uint16_t* sin_tab, int64_t pos0, uint16_t* q_out,
                                  int8_t* kc, uint16_t* ks, int8_t* vc, uint16_t* vs,
                                  int64_t code_head_stride, int64_t s_len, uint16_t* k_f16,
                                  uint16_t* v_f16, int64_t f16_head_stride, float clip_qkv,
                                  void* stream);

/* Causal attention over T prompt rows (HF OlmoeAttention with sdpa, the
 * reference's multi-token path, src/lemoq/kernels/attn_decode.py:836-1017):
 * out[t, h, :] = softmax over keys j <= t of (q_t . k_j) * scale, times v_j;
 * qk_scale = scale * log2(e); fp32 statistics, fp16 out.
 *   q (T, q_ld) with head h at column h*D; k, v (heads, kv_head_stride) with
 *   key j of head h at h*kv_head_stride + j*D; out (T, out_ld).
 *   D in {64, 128, 256}; q, k, v 16-byte aligned, out 8-byte aligned. */
int lemoq_attn_prefill_f16(const uint16_t* q, int64_t q_ld, const uint16_t* k, const uint16_t* v,
                           int64_t kv_head_stride, int64_t T, int64_t heads, int64_t head_dim,
                           float qk_scale, uint16_t* out, int64_t out_ld, void* stream);

/* MoE block of several tokens (replaces _prefill_forward,
 * src/lemoq/kernels/moe_static.py:329-371, for quantized experts: each
 * expert's weights read once for all of its tokens).
 * Tile table size for `pairs` = T*top_k (token, slot) pairs and E experts. */
int64_t lemoq_moe_prefill_max_tiles(int64_t pairs, int64_t E);

/* Stable sort of the pairs by expert: pair_tok/pair_src/pair_w (T*top_k)
 * hold, in expert order and token order within an expert, the token, the
 * pair index token*top_k + slot and fp16(top_w); expert_off (E+1) the run
 * starts; tiles (max_tiles, 4) int32 rows (expert, begin, end, 0) of at most
 * 128 pairs, unused rows with expert -1.  top_i (T, top_k) int64 in [0, E),
 * top_w (T, top_k) fp32 (lemoq_route_topk's outputs).  E <= 255,
 * top_k <= 8, T*top_k <= 32768. */
int lemoq_moe_prefill_sort(const int64_t* top_i, const float* top_w, int64_t T, int64_t top_k,
                           int64_t E, int32_t* pair_tok, int32_t* pair_src, uint16_t* pair_w,
                           int32_t* expert_off, int32_t* tiles, int64_t max_tiles, void* stream);

/* act (pairs, F) = fp16(fp16(silu(g)) * u), g and u the fp16 outputs of
 * x[pair_tok] @ w^T for the expert's gate rows [0, F) and up rows [F, 2F)
 * (w8, w = fp16(code * scale)).  x (T, H) fp16; gu_codes (E, 2F, H) int8;
 * gu_scale (E, 2F, H/group) fp16.  H, F and group multiples of 64. */
int lemoq_moe_prefill_gate_up(const uint16_t* x, int64_t H, const int32_t* pair_tok,
                              const int32_t* tiles, int64_t max_tiles, const int8_t* gu_codes,
                              const uint16_t* gu_scale, int64_t F, int64_t group, uint16_t* act,
                              void* stream);

/* y[pair_src] (H) = fp16(fp16(act @ w_down^T) * pair_w) for each sorted pair.
 * dn_codes (E, H, F) int8; dn_scale (E, H, F/group) fp16; y (T*top_k, H), 16-byte
 * aligned (the rows are written in 16-byte chunks). */
int lemoq_moe_prefill_down(const uint16_t* act, int64_t F, const int32_t* pair_src,
                           const uint16_t* pair_w, const int32_t* tiles, int64_t max_tiles,
                           const int8_t* dn_codes, const uint16_t* dn_scale, int64_t H,
                           int64_t group, uint16_t* y, void* stream);

/* out[t] = fp16(residual[t] + s), s the fp16 running sum (from 0) of the
 * token's y rows in ascending expert order (the order the reference's expert
 * loop index_adds them); residual nullable (then out = s), may alias out.
 * H % 8 == 0; y, out, residual 16-byte aligned. */
int lemoq_moe_prefill_combine(const uint16_t* y, const int64_t* top_i, int64_t T, int64_t top_k,
                              int64_t H, const uint16_t* residual, uint16_t* out, void* stream);

/* lemoq_moe_prefill_combine, and in the same launch xn_out[t] = the RMSNorm
 * of out[t] with norm_w (the next decoder layer's input_layernorm, rounded as
 * lemoq_rmsnorm rounds it on 16-byte aligned rows, bit for bit: the same sum
 * order of the squares).  H <= 8192; norm_w and xn_out 16-byte aligned too
 * (the norm reads and writes 16-byte chunks); xn_out (T, H) must not overlap
 * y, residual or out. */
int lemoq_moe_prefill_combine_norm(const uint16_t* y, const int64_t* top_i, int64_t T, int64_t top_k,
                                   int64_t H, const uint16_t* residual, uint16_t* out,
                                   const uint16_t* norm_w, float eps, uint16_t* xn_out, void* stream);

/* ---------------------------------------------------------------------------
 * Measurement: read n_bytes (multiple of 16, 16-byte aligned) once with
 * nontemporal 16-byte loads.  The buffer is cut into contiguous shares of
 * per = ceil(n_bytes / blocks) bytes rounded up to 4 KB; block b (one per
 * non-empty share, at most `blocks`) reads share b in 4 KB wave chunks and
 * writes a fold of what it read to out[b] (out holds `blocks` entries; those
 * past the last non-empty share are left untouched).  The roofline
 * denominator (measured read bandwidth) and the cache flush before cold kernel
 * timings.  Restates the method of the reference's read probe
 * (tools/probe_machine.py:392-505).
 * ------------------------------------------------------------------------- */
int lemoq_read_probe(const void* src, int64_t n_bytes, uint32_t* out, int64_t blocks,
                     void* stream);

/* Measurement: copy n_bytes (multiple of 16, both pointers 16-byte aligned,
 * no overlap) from src to dst with 16-byte loads and stores over `blocks`
 * 256-thread blocks.  A kernel of known traffic (n_bytes read, n_bytes
 * written) that calibrates the profiler's FETCH_SIZE and WRITE_SIZE counters
 * before they are read as HBM bytes of the step's kernels.  No counterpart in
 * the reference (its profiling reads wall time only).
 * ------------------------------------------------------------------------- */
int lemoq_copy_probe(const void* src, void* dst, int64_t n_bytes, int64_t blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LEMOQ_HIP_H */
