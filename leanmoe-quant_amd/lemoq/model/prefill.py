"""Batched prompt prefill of the OLMoE W8 model on the matrix cores.

The reference's session prefills the whole prompt with one forward of the
patched HF model (``StaticCacheDecodeSession.prefill``,
``benchmarks/cudagraph.py:578-599``).  With more than one token every patched
operator takes its multi-token branch, and this module runs exactly that path
with the HIP kernels, one layer at a time:

=====================  ==========================================================
HF / reference         here (C-ABI entry point)
=====================  ==========================================================
embed_tokens           ``lemoq_gather_rows``
input_layernorm        ``lemoq_rmsnorm`` (the fused RMSNorm, any row count) for layer 0;
                       the previous layer's ``lemoq_moe_prefill_combine_norm`` after
q/k/v_proj             ``lemoq_gemm_w8`` (QuantLinear separate arm, linear.py:471-480)
q_norm, k_norm, RoPE,  ``lemoq_qk_norm_rope_kv_i8_rows`` (HF RoPE rounding; the
KV cache + INT8 bulk   KV-INT8 rows are what kv_int8_bulk_quantize gives)
sdpa causal attention  ``lemoq_attn_prefill_f16``; in the last layer only the last
                       query: ``lemoq_attn_split_f16`` + ``lemoq_attn_merge`` (nothing
                       after the last layer reads another position, so its
                       attention, o_proj, norm, router and MoE run on that row)
o_proj + residual      ``lemoq_gemm_w8`` with the residual in its epilogue
post_attention norm    ``lemoq_rmsnorm``
router F.linear +      ``lemoq_gemm_f16_splitk`` (fp32 partials only);
routing_softmax_topk   ``lemoq_route_topk_splitk`` (sums the partials, then routes)
_prefill_forward       ``lemoq_moe_prefill_sort`` / ``_gate_up`` / ``_down`` /
(moe_static.py:329)    ``_combine`` (the combine adds the residual; ``_combine_norm``
                       also writes the next layer's input norm)
final norm, lm_head,   ``lemoq_lm_head_argmax_w8_dq`` on the last row: the final
greedy pick            norm in the GEMV's prologue, weights rounded to fp16 before
                       the dot (the separate arm's arithmetic), then the argmax
=====================  ==========================================================

The KV-INT8 cache slots 0..T-1 of every layer are written; the logits of the
last prompt position land in ``logits`` and their greedy pick in ``step["token"]``.  All launches go on torch's current
stream; scratch tensors are allocated per call (prefill is eager, as in the
reference).
"""

from __future__ import annotations

import math
from typing import Any

import torch

from lemoq import _hip

__all__ = ["prefill_prompt", "PREFILL_MAX_PAIRS"]

LOG2E = 1.4426950408889634
# T * top_k pairs are sorted in one block's LDS (lemoq_moe_prefill_sort).
PREFILL_MAX_PAIRS = 32768


def prefill_prompt(weights: Any, tokens: Any, kv: list, cos_tab: Any, sin_tab: Any, max_seq: int,
                   logits: Any, step: dict | None = None, last_row_only: bool = True,
                   kv_f16: list | None = None) -> None:
    """Prefill ``tokens`` (int64 (T,) on the device) at positions 0..T-1.

    ``kv``: per layer the KV-INT8 cache dict (kc (heads, S, D) int8, ks (heads, S)
    fp16, vc, vs), or the fp16 cache dict (k, v (heads, S, D) fp16: KV-INT8 off,
    the rows written as they are), with S = ``max_seq``; ``cos_tab``/``sin_tab``
    (S, D) fp16;
    ``logits`` (vocab,) fp16 receives the last position's logits.  ``step``: the
    decode session's device state that the greedy pick advances, as
    ``lemoq_argmax_advance`` does (``token``, ``pos`` holding T - 1, ``filled``,
    ``history``; the prompt is ``tokens``); scratch buffers when None.
    ``last_row_only``: run the last layer after its KV rows on the last position
    only (the default; False runs it on every position, as the other layers).
    ``kv_f16``: when a list, receives per layer copies of the fp16 k (after k_norm
    and RoPE) and v rows that were written (or quantised) into the cache, each
    (heads, T, D) (for parity checks of the KV bytes against their inputs).
    """
    s = weights.shape
    dev = weights.device
    T = int(tokens.numel())
    S = int(max_seq)
    H, NH, D, E, K, F = s.hidden, s.heads, s.head_dim, s.num_experts, s.top_k, s.ffn
    HD = NH * D
    g = s.group_size
    if T < 1 or T > S:
        raise ValueError("prompt length %d outside [1, %d]" % (T, S))
    if T * K > PREFILL_MAX_PAIRS:
        raise NotImplementedError("prefill sorts at most %d (token, expert) pairs; T*top_k = %d"
                                  % (PREFILL_MAX_PAIRS, T * K))
    if tokens.dtype != torch.int64 or tokens.device != dev or not tokens.is_contiguous():
        raise ValueError("tokens must be a contiguous int64 tensor on %s" % dev)
    _hip.require_rocm(tokens, weights.embed, what="prefill_prompt")
    lib = _hip.load()
    P = _hip.ptr
    st = _hip.stream_of(dev)
    f16 = dict(dtype=torch.float16, device=dev)
    i32 = dict(dtype=torch.int32, device=dev)

    h = torch.empty((T, H), **f16)
    xn = torch.empty((T, H), **f16)
    qkv = torch.empty((T, 3 * HD), **f16)
    q = torch.empty((T, HD), **f16)
    fp16_cache = "k" in kv[0]
    if not fp16_cache:  # fp16 rows for the prompt's attention, then quantised into the cache
        k16 = torch.empty((NH, S, D), **f16)
        v16 = torch.empty((NH, S, D), **f16)
    attn = torch.empty((T, HD), **f16)
    # the router's 64 outputs give few output tiles: K is cut into up to 8 ranges
    # whose fp32 partials the routing launch sums; fp16 logits only without a split
    rsplit = next(sp for sp in (8, 4, 2, 1) if H % (64 * sp) == 0)
    rlog = torch.empty((T, E), **f16) if rsplit == 1 else None
    rws = torch.empty((rsplit, T, E), dtype=torch.float32, device=dev)
    top_w = torch.empty((T, K), dtype=torch.float32, device=dev)
    top_i = torch.empty((T, K), dtype=torch.int64, device=dev)
    pairs = T * K
    max_tiles = int(lib.lemoq_moe_prefill_max_tiles(pairs, E))
    pair_tok = torch.empty((pairs,), **i32)
    pair_src = torch.empty((pairs,), **i32)
    pair_w = torch.empty((pairs,), **f16)
    expert_off = torch.empty((E + 1,), **i32)
    tiles = torch.empty((max_tiles, 4), **i32)
    act = torch.empty((pairs, F), **f16)
    ybuf = torch.empty((pairs, H), **f16)
    qk_scale = float((1.0 / math.sqrt(D)) * LOG2E)

    _hip.call("lemoq_gather_rows", P(weights.embed), s.vocab, H, P(tokens), T, P(h), st)
    _hip.call("lemoq_rmsnorm", P(h), T, H, P(weights.layers[0].ln_in), float(s.eps), P(xn), st)
    n_layers = len(weights.layers)
    for li, (L, c) in enumerate(zip(weights.layers, kv)):
        # xn holds this layer's input norm: the previous layer's combine wrote it
        _hip.call("lemoq_gemm_w8", P(xn), T, H, H, None, P(L.qkv_codes), P(L.qkv_scale), 3 * HD, g,
                  P(qkv), 3 * HD, None, 0, st)
        if fp16_cache:  # the cache is the attention's k/v (no KV-INT8 rows)
            k16, v16 = c["k"], c["v"]
            i8 = (None, None, None, None)
        else:
            i8 = (P(c["kc"]), P(c["ks"]), P(c["vc"]), P(c["vs"]))
        _hip.call("lemoq_qk_norm_rope_kv_i8_rows", P(qkv), T, NH, D, P(L.q_norm), P(L.k_norm), float(s.eps),
                  P(cos_tab), P(sin_tab), 0, P(q), *i8, S * D, S,
                  P(k16), P(v16), S * D, math.inf if s.clip_qkv is None else float(s.clip_qkv), st)
        if kv_f16 is not None:
            kv_f16.append((k16[:, :T].clone(), v16[:, :T].clone()))
        if li + 1 == n_layers and T > 1 and last_row_only:
            _last_layer_last_row(L, T, q, k16, v16, h, xn, attn, rws, rsplit, rlog, top_w, top_i, pair_tok,
                                 pair_src, pair_w, expert_off, tiles, act, ybuf, s, S, qk_scale, lib, st)
            break
        _hip.call("lemoq_attn_prefill_f16", P(q), HD, P(k16), P(v16), S * D, T, NH, D, qk_scale, P(attn), HD, st)
        _hip.call("lemoq_gemm_w8", P(attn), T, HD, HD, None, P(L.o_codes), P(L.o_scale), H, g, P(h), H, P(h), H,
                  st)
        _hip.call("lemoq_rmsnorm", P(h), T, H, P(L.ln_post), float(s.eps), P(xn), st)
        if rsplit > 1:  # partials only; the routing launch sums them as the GEMM's finish would
            _hip.call("lemoq_gemm_f16_splitk", P(xn), T, H, H, P(L.router), E, None, E, rsplit, P(rws), st)
            _hip.call("lemoq_route_topk_splitk", P(rws), rsplit, T, E, K, int(bool(s.norm_topk_prob)), P(top_w),
                      P(top_i), st)
        else:
            _hip.call("lemoq_gemm_f16_splitk", P(xn), T, H, H, P(L.router), E, P(rlog), E, 1, P(rws), st)
            _hip.call("lemoq_route_topk", P(rlog), 1, T, E, E, K, int(bool(s.norm_topk_prob)), P(top_w), P(top_i),
                      st)
        _hip.call("lemoq_moe_prefill_sort", P(top_i), P(top_w), T, K, E, P(pair_tok), P(pair_src), P(pair_w),
                  P(expert_off), P(tiles), max_tiles, st)
        _hip.call("lemoq_moe_prefill_gate_up", P(xn), H, P(pair_tok), P(tiles), max_tiles, P(L.gu_codes),
                  P(L.gu_scale), F, g, P(act), st)
        _hip.call("lemoq_moe_prefill_down", P(act), F, P(pair_src), P(pair_w), P(tiles), max_tiles,
                  P(L.dn_codes), P(L.dn_scale), H, g, P(ybuf), st)
        if li + 1 < n_layers:
            _hip.call("lemoq_moe_prefill_combine_norm", P(ybuf), P(top_i), T, K, H, P(h), P(h),
                      P(weights.layers[li + 1].ln_in), float(s.eps), P(xn), st)
        else:
            _hip.call("lemoq_moe_prefill_combine", P(ybuf), P(top_i), T, K, H, P(h), P(h), st)
    if step is None:
        step = {"token": torch.zeros((1,), dtype=torch.int64, device=dev),
                "pos": torch.full((1,), T - 1, dtype=torch.int64, device=dev),
                "filled": torch.zeros((1,), dtype=torch.int32, device=dev),
                "history": torch.zeros((T + 1,), dtype=torch.int64, device=dev)}
    parts = int(lib.lemoq_lm_head_argmax_parts(s.vocab))
    part_val = torch.empty((parts,), dtype=torch.float32, device=dev)
    part_idx = torch.empty((parts,), dtype=torch.int32, device=dev)
    lm_f16 = getattr(weights, "lm_f16", None)
    if lm_f16 is not None:
        # fp16 lm_head (F.linear in fp16 on the normed last row), then the greedy pick
        _hip.call("lemoq_lm_head_argmax_f16", P(h[T - 1:]), P(weights.final_norm), float(s.eps), P(lm_f16), s.vocab,
                  H, P(logits), P(part_val), P(part_idx), parts, P(step["token"]), P(step["pos"]), P(step["filled"]),
                  P(tokens), T, P(step["history"]), int(step["history"].numel()), st)
        return
    _hip.call("lemoq_lm_head_argmax_w8_dq", P(h[T - 1:]), P(weights.final_norm), float(s.eps), P(weights.lm_codes),
              P(weights.lm_scale), s.vocab, H, g, P(logits), P(part_val), P(part_idx), parts, P(step["token"]),
              P(step["pos"]), P(step["filled"]), P(tokens), T, P(step["history"]), int(step["history"].numel()), st)
    # The scratch tensors are released when this returns; the caching allocator
    # hands their memory only to later work on this same stream, which runs
    # after these kernels.


def _last_layer_last_row(L: Any, T: int, q: Any, k16: Any, v16: Any, h: Any, xn: Any, attn: Any, rws: Any,
                         rsplit: int, rlog: Any, top_w: Any, top_i: Any, pair_tok: Any, pair_src: Any, pair_w: Any,
                         expert_off: Any, tiles: Any, act: Any, ybuf: Any, s: Any, S: int, qk_scale: float,
                         lib: Any, st: Any) -> None:
    """The last layer after its KV rows are written, for the last position only.

    Nothing after the last layer reads another position: the prefill returns the
    last position's logits and its greedy pick, and every layer's KV-INT8 rows are
    already in the cache.  So the last layer's attention runs for the one query at
    T - 1 over keys 0..T-1 (the decode split-KV fp16 kernel and its merge, on the
    fp16 K/V rows the prologue just wrote), and o_proj + residual, the post norm,
    the router and the MoE block (sort, grouped gate/up and down, combine) run on
    that row with the same kernels as the other layers.
    """
    P = _hip.ptr
    H, NH, D, E, K, F = s.hidden, s.heads, s.head_dim, s.num_experts, s.top_k, s.ffn
    HD, g, dev = NH * D, s.group_size, q.device
    from lemoq.model.olmoe import step_num_splits  # noqa: PLC0415

    ns = step_num_splits(T, NH)
    m = torch.empty((NH * ns,), dtype=torch.float32, device=dev)
    ls = torch.empty_like(m)
    acc = torch.empty((NH * ns * D,), dtype=torch.float32, device=dev)
    filled = torch.full((1,), T, dtype=torch.int32, device=dev)
    hl = h[T - 1:]
    _hip.call("lemoq_attn_split_f16", P(q[T - 1:]), P(k16), P(v16), S * D, P(filled), NH, D, ns, qk_scale, P(m),
              P(ls), P(acc), st)
    _hip.call("lemoq_attn_merge", P(m), P(ls), P(acc), NH, ns, D, P(attn), st)
    _hip.call("lemoq_gemm_w8", P(attn), 1, HD, HD, None, P(L.o_codes), P(L.o_scale), H, g, P(hl), H, P(hl), H, st)
    _hip.call("lemoq_rmsnorm", P(hl), 1, H, P(L.ln_post), float(s.eps), P(xn), st)
    norm = int(bool(s.norm_topk_prob))
    if rsplit > 1:
        _hip.call("lemoq_gemm_f16_splitk", P(xn), 1, H, H, P(L.router), E, None, E, rsplit, P(rws), st)
        _hip.call("lemoq_route_topk_splitk", P(rws), rsplit, 1, E, K, norm, P(top_w), P(top_i), st)
    else:
        _hip.call("lemoq_gemm_f16_splitk", P(xn), 1, H, H, P(L.router), E, P(rlog), E, 1, P(rws), st)
        _hip.call("lemoq_route_topk", P(rlog), 1, 1, E, E, K, norm, P(top_w), P(top_i), st)
    mt = int(lib.lemoq_moe_prefill_max_tiles(K, E))
    _hip.call("lemoq_moe_prefill_sort", P(top_i), P(top_w), 1, K, E, P(pair_tok), P(pair_src), P(pair_w),
              P(expert_off), P(tiles), mt, st)
    # one token meets each of its top_k experts once: the sort's live tiles are
    # the first top_k entries of the table (the rest marked unused)
    _hip.call("lemoq_moe_prefill_gate_up", P(xn), H, P(pair_tok), P(tiles), K, P(L.gu_codes), P(L.gu_scale), F, g,
              P(act), st)
    _hip.call("lemoq_moe_prefill_down", P(act), F, P(pair_src), P(pair_w), P(tiles), K, P(L.dn_codes),
              P(L.dn_scale), H, g, P(ybuf), st)
    _hip.call("lemoq_moe_prefill_combine", P(ybuf), P(top_i), 1, K, H, P(hl), P(hl), st)
