"""CPU decode step of the OLMoE w8a16 + W8 lm_head + KV-INT8 cell.

Test infrastructure (see ``oracle/__init__.py``).  ``OracleDecoder.step``
restates, on CPU tensors, the HF OLMoE decoder (transformers
``OlmoeModel``/``OlmoeDecoderLayer``/``OlmoeAttention``/``OlmoeSparseMoeBlock``)
as patched by the reference's canonical cell:

* packed q|k|v via the fused w8 GEMV (``src/lemoq/kernels/packed_qkv.py:78-96``);
  q_norm/k_norm over heads*D, fused RoPE (``rope.py:154-203``);
* KV-INT8 write of the new row then split-KV INT8 attention over
  ``[0, pos+1)`` (``attn_decode.py:952-1000``, ``kv_int8.py:223-257``); or, with
  ``kv_cache="fp16"`` (KV-INT8 off), the fp16 row written as it is
  (``kv_direct_write``, ``attn_decode.py:930-948``) and the fp16 split-KV
  attention over ``[0, pos+1)`` (``attn_decode.py:999-1008``);
* o_proj, fp16 residual add; post-attention norm; ``_route``; grouped w8 MoE
  (``moe_grouped_quant.py:562-601``); fp16 residual add;
* final norm, W8 lm_head; greedy argmax (first index on ties).

Weights come as plain CPU tensors with the same field names as
``lemoq.model.olmoe.OlmoeW8Weights``.  Static weights (q|k|v, o, lm_head) are
dequantised once; experts are dequantised when selected.  ``bits`` 4 (the
reference's w4a16 cell: 4-bit symmetric codes of attention and experts,
packed two per byte, the even column in the low nibble) unpacks the codes
with ``oracle.quant.unpack_4bit`` first and computes ``code * scale`` as for
8 bits; ``lm_f16`` (the reference's fp16 lm_head of every cell but w8a16 with
its lm_head switch on, ``benchmarks/runner.py:393-412``) replaces the W8
lm_head by an fp16 ``F.linear`` (fp32 accumulation, one fp16 rounding).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from oracle import ops
from oracle import quant as oq

LOG2E = 1.4426950408889634


@dataclass(frozen=True)
class Shape:
    hidden: int = 2048
    heads: int = 16
    head_dim: int = 128
    layers: int = 16
    num_experts: int = 64
    top_k: int = 8
    ffn: int = 1024
    vocab: int = 50304
    eps: float = 1e-5
    rope_theta: float = 10000.0
    norm_topk_prob: bool = False
    group_size: int = 128
    init_std: float = 0.02
    clip_qkv: float | None = None


@dataclass
class HostLayer:
    ln_in: Any
    ln_post: Any
    q_norm: Any
    k_norm: Any
    qkv_codes: Any
    qkv_scale: Any
    o_codes: Any
    o_scale: Any
    router: Any
    gu_codes: Any
    gu_scale: Any
    dn_codes: Any
    dn_scale: Any


@dataclass
class HostWeights:
    shape: Any
    embed: Any
    final_norm: Any
    lm_codes: Any
    lm_scale: Any
    layers: list = field(default_factory=list)
    bits: int = 8          # attention and expert code width (4: packed two per byte)
    lm_f16: Any = None     # fp16 lm_head (vocab, H) in place of lm_codes / lm_scale


def random_host_weights(shape: Shape, seed: int = 0, *, bits: int = 8, lm_head: str = "w8") -> HostWeights:
    """Seeded CPU init for tiny CPU-only oracle tests (numpy RTN; not the device
    generator).  ``bits`` 4 quantises attention and experts to packed 4-bit
    symmetric codes; ``lm_head`` "fp16" keeps the lm_head in fp16."""
    if bits not in (4, 8) or lm_head not in ("w8", "fp16"):
        raise ValueError("bits must be 4 or 8 and lm_head 'w8' or 'fp16'")
    g = torch.Generator().manual_seed(seed)
    s = shape
    HD = s.heads * s.head_dim

    def normal(*size: int) -> Any:
        return torch.randn(size, generator=g, dtype=torch.float32) * s.init_std

    def gamma(n: int) -> Any:
        return (torch.rand((n,), generator=g, dtype=torch.float32) + 0.5).to(torch.float16)

    def q8_lm(w: Any):
        q = oq.rtn_quantize_w8(w.numpy(), s.group_size)
        return torch.from_numpy(q["codes_padded"]), torch.from_numpy(q["scale_f16"])

    def q8(w: Any):
        if bits == 8:
            return q8_lm(w)
        q = oq.rtn_quantize(w.numpy(), bits=4, group_size=s.group_size, symmetric=True)
        return torch.from_numpy(oq.pack_4bit(q["codes_padded"])), torch.from_numpy(q["scale_f16"])

    embed = normal(s.vocab, s.hidden).to(torch.float16)
    layers = []
    for _ in range(s.layers):
        ln_in, ln_post, qn, kn = gamma(s.hidden), gamma(s.hidden), gamma(HD), gamma(HD)
        qkv_c, qkv_s = q8(normal(3 * HD, s.hidden))
        o_c, o_s = q8(normal(s.hidden, HD))
        router = normal(s.num_experts, s.hidden).to(torch.float16)
        gu_c, gu_s = q8(normal(s.num_experts * 2 * s.ffn, s.hidden))
        dn_c, dn_s = q8(normal(s.num_experts * s.hidden, s.ffn))
        per = 8 // bits  # codes per byte
        layers.append(HostLayer(
            ln_in=ln_in, ln_post=ln_post, q_norm=qn, k_norm=kn, qkv_codes=qkv_c, qkv_scale=qkv_s,
            o_codes=o_c, o_scale=o_s, router=router,
            gu_codes=gu_c.reshape(s.num_experts, 2 * s.ffn, s.hidden // per),
            gu_scale=gu_s.reshape(s.num_experts, 2 * s.ffn, s.hidden // s.group_size),
            dn_codes=dn_c.reshape(s.num_experts, s.hidden, s.ffn // per),
            dn_scale=dn_s.reshape(s.num_experts, s.hidden, s.ffn // s.group_size),
        ))
    final_norm = gamma(s.hidden)
    lm = normal(s.vocab, s.hidden)
    if lm_head == "fp16":
        return HostWeights(shape=s, embed=embed, final_norm=final_norm, lm_codes=None, lm_scale=None,
                           layers=layers, bits=bits, lm_f16=lm.to(torch.float16))
    lm_c, lm_s = q8_lm(lm)
    return HostWeights(shape=s, embed=embed, final_norm=final_norm, lm_codes=lm_c, lm_scale=lm_s, layers=layers,
                       bits=bits)


def unpacked_codes(codes: Any, bits: int) -> Any:
    """The codes as int8 values: 8-bit codes as they are, 4-bit ones unpacked
    (``oracle.quant.unpack_4bit``, signed, low nibble first)."""
    if int(bits) == 8:
        return codes
    return torch.from_numpy(oq.unpack_4bit(codes.numpy(), signed=True))


def lm_head_weight(weights: Any) -> Any:
    """The lm_head as fp32 values: the fp16 lm_head, or the W8 one dequantised."""
    lm_f16 = getattr(weights, "lm_f16", None)
    if lm_f16 is not None:
        return lm_f16.to(torch.float32)
    return ops.dequant_w8(weights.lm_codes, weights.lm_scale, weights.shape.group_size)


class OracleDecoder:
    """CPU decode step with its own KV cache of ``max_seq`` slots: KV-INT8 (kc, ks,
    vc, vs per layer) or, with ``kv_cache="fp16"``, fp16 rows (k, v per layer).  A
    ``kv`` list given in either form sets the kind."""

    def __init__(self, weights: Any, max_seq: int, *, kv: list | None = None, kv_cache: str = "int8") -> None:
        self.w = weights
        s = weights.shape
        self.s = s
        self.max_seq = int(max_seq)
        g = s.group_size
        self.bits = int(getattr(weights, "bits", 8))
        if self.bits not in (4, 8):
            raise ValueError("weights.bits must be 4 or 8")
        self.qkv_w = [ops.dequant_w8(unpacked_codes(L.qkv_codes, self.bits), L.qkv_scale, g) for L in weights.layers]
        self.o_w = [ops.dequant_w8(unpacked_codes(L.o_codes, self.bits), L.o_scale, g) for L in weights.layers]
        self.lm_w = lm_head_weight(weights)
        cos, sin = ops.rotary_cos_sin(torch.arange(self.max_seq), s.head_dim, s.rope_theta)
        self.cos, self.sin = cos, sin
        if kv is not None:
            kv_cache = "fp16" if "k" in kv[0] else "int8"
        if kv_cache not in ("int8", "fp16"):
            raise ValueError("kv_cache must be 'int8' or 'fp16', got %r" % (kv_cache,))
        self.kv_cache = kv_cache
        if kv is None and kv_cache == "fp16":
            kv = [
                {
                    "k": torch.zeros((s.heads, self.max_seq, s.head_dim), dtype=torch.float16),
                    "v": torch.zeros((s.heads, self.max_seq, s.head_dim), dtype=torch.float16),
                }
                for _ in range(s.layers)
            ]
        if kv is None:
            kv = [
                {
                    "kc": torch.zeros((s.heads, self.max_seq, s.head_dim), dtype=torch.int8),
                    "ks": torch.ones((s.heads, self.max_seq), dtype=torch.float16),
                    "vc": torch.zeros((s.heads, self.max_seq, s.head_dim), dtype=torch.int8),
                    "vs": torch.ones((s.heads, self.max_seq), dtype=torch.float16),
                }
                for _ in range(s.layers)
            ]
        self.kv = kv
        self.trace: dict[str, Any] = {}

    @staticmethod
    def _linear(x16: Any, w32: Any) -> Any:
        """fused w8 GEMV numerics: fp32 accumulate, one fp16 rounding."""
        return (x16.to(torch.float32).reshape(1, -1) @ w32.t()).reshape(-1).to(torch.float16)

    def _quant_into(self, cache_c: Any, cache_s: Any, pos: int, rows16: Any) -> None:
        codes, scales = oq.kv_quantize_rows(rows16.numpy())
        cache_c[:, pos, :] = torch.from_numpy(codes)
        cache_s[:, pos] = torch.from_numpy(scales)

    def step(self, token: int, pos: int, *, keep_trace: bool = False) -> Any:
        """Process ``token`` at position ``pos``; returns the fp16 logits (vocab,)."""
        s, w = self.s, self.w
        H, NH, D = s.hidden, s.heads, s.head_dim
        HD = NH * D
        if not (0 <= pos < self.max_seq):
            raise ValueError("pos outside the cache")
        qk_scale = (1.0 / math.sqrt(D))
        h = w.embed[int(token)].clone()
        cos, sin = self.cos[pos], self.sin[pos]
        for li, L in enumerate(w.layers):
            kv = self.kv[li]
            r = h
            xn = ops.rms_norm(h, L.ln_in, s.eps)
            qkv = self._linear(xn, self.qkv_w[li])
            q, k, v = qkv[:HD], qkv[HD : 2 * HD], qkv[2 * HD :]
            q = ops.rms_norm(q, L.q_norm, s.eps)
            k = ops.rms_norm(k, L.k_norm, s.eps)
            q, k, v = ops.clip_qkv(q, k, v, getattr(s, "clip_qkv", None))
            q = ops.rope_fused(q.reshape(NH, D), cos, sin)
            k = ops.rope_fused(k.reshape(NH, D), cos, sin)
            if self.kv_cache == "fp16":
                kv["k"][:, pos, :] = k
                kv["v"][:, pos, :] = v.reshape(NH, D)
                attn = ops.split_kv_oracle(q, kv["k"], kv["v"], pos + 1, num_splits=1,
                                           scale=qk_scale).to(torch.float16).reshape(-1)
            else:
                self._quant_into(kv["kc"], kv["ks"], pos, k)
                self._quant_into(kv["vc"], kv["vs"], pos, v.reshape(NH, D))
                attn = ops.int8_attention_folded(q, kv["kc"], kv["ks"], kv["vc"], kv["vs"], pos + 1,
                                                 scale=qk_scale).to(torch.float16).reshape(-1)
            o = self._linear(attn, self.o_w[li])
            h = r + o
            r = h
            xn = ops.rms_norm(h, L.ln_post, s.eps)
            logits_r, top_w, top_i = ops.route(xn.reshape(1, -1), L.router, s.top_k, s.norm_topk_prob)
            ids = top_i.reshape(-1)
            if self.bits == 8:
                moe, act = ops.grouped_moe_w8(xn, L.gu_codes, L.gu_scale, L.dn_codes, L.dn_scale,
                                              s.group_size, ids, top_w.reshape(-1))
            else:  # the selected experts' codes unpacked; slot i reads row i of them
                moe, act = ops.grouped_moe_w8(xn, unpacked_codes(L.gu_codes[ids], 4), L.gu_scale[ids],
                                              unpacked_codes(L.dn_codes[ids], 4), L.dn_scale[ids],
                                              s.group_size, torch.arange(ids.numel()), top_w.reshape(-1))
            h = r + moe
            if keep_trace:
                self.trace.setdefault("top_i", []).append(top_i.reshape(-1).clone())
                self.trace.setdefault("h", []).append(h.clone())
        hn = ops.rms_norm(h, w.final_norm, s.eps)
        return self._linear(hn, self.lm_w)

    def greedy(self, logits: Any) -> int:
        """First index of the maximum (``torch.argmax``/``.item()`` of the reference session)."""
        lf = logits.to(torch.float32).numpy()
        return int(np.argmax(lf))

    def run(self, prompt: list[int], new_tokens: int, *, start_pos: int = 0, seed_token: int | None = None):
        """Prefill ``prompt`` by stepping it (positions start_pos..), then ``new_tokens`` greedy steps.

        Returns ``(tokens, logits_per_decode_step)``; ``tokens[0]`` is the seed token.
        """
        pos = start_pos
        logits = None
        for t in prompt:
            logits = self.step(int(t), pos)
            pos += 1
        tok = self.greedy(logits) if seed_token is None else int(seed_token)
        tokens, all_logits = [tok], []
        for _ in range(new_tokens):
            logits = self.step(tok, pos)
            all_logits.append(logits)
            pos += 1
            tok = self.greedy(logits)
            tokens.append(tok)
        return tokens, all_logits


def oracle_prefill(weights: Any, tokens: Any, max_seq: int, *, all_logits: bool = False,
                   kv_f16: list | None = None, kv_layers: int | None = None, kv_cache: str = "int8"):
    """The reference's prefill of the prompt ``tokens`` (positions 0..T-1) on the CPU.

    ``StaticCacheDecodeSession.prefill`` (``benchmarks/cudagraph.py:578-599``) runs the
    patched HF model over all T tokens at once; every patched operator takes its
    multi-token branch there:

    * linears: ``QuantLinear`` "separate" arm, fp16 weight then ``F.linear``
      (``src/lemoq/quant/linear.py:365-395,420-434,471-480``) -> ``ops.linear_separate_w8``;
    * RMSNorms (input, q/k over heads*D, post-attention, final): the fused kernel for any
      row count (``rmsnorm.py:102-163``) -> ``ops.rms_norm``;
    * RoPE: HF ``apply_rotary_pos_emb`` (the fused RoPE guard takes q_len == 1 only,
      ``rope.py:140-177``) -> ``ops.rope_hf``;
    * attention: HF's own forward with sdpa and a causal mask (the decode core is only
      taken for q_len == 1, ``attn_decode.py:836-1017``) -> ``ops.causal_attention``;
    * MoE: router ``F.linear`` in fp16, ``_route``, per-expert loop
      (``moe_static.py:262-283,329-371``) -> ``ops.linear_f16``, ``ops.route_logits``,
      ``ops.moe_prefill_w8``;
    * the KV-INT8 cache is the bulk quantisation of the fp16 k/v rows
      (``kv_int8.py:127-162``) -> ``oracle.quant.kv_quantize_rows``; with
      ``kv_cache="fp16"`` (KV-INT8 off) the cache holds those fp16 rows;
    * logits: final norm and the W8 lm_head (separate arm: T > 1 rows reach it), or the
      fp16 lm_head (``lm_f16``) as an fp16 ``F.linear``;
    * 4-bit weights (``bits`` 4, the w4a16 cell): the codes unpacked, then the same
      separate arm (``code * scale`` rounded to fp16).

    Returns ``(logits, kv)``: fp16 logits of the last position (``(T, vocab)`` with
    ``all_logits``), and per layer the KV-INT8 cache dict (kc, ks, vc, vs) of ``max_seq``
    slots with slots 0..T-1 filled (the rest codes 0, scales 1), or the fp16 cache dict
    (k, v; the rest zeros).  ``kv_f16``, when a
    list, receives per layer the fp16 k (after k_norm and RoPE) and v rows that were
    quantised, each (heads, T, D).  ``kv_layers`` stops after that many layers' KV rows
    (logits are then None).
    """
    s, w = weights.shape, weights
    bits = int(getattr(weights, "bits", 8))  # 4: the w4a16 cell, codes unpacked before the separate arm
    toks = torch.as_tensor(tokens, dtype=torch.int64).reshape(-1)
    T = int(toks.numel())
    NH, D = s.heads, s.head_dim
    HD = NH * D
    g = s.group_size
    if not (0 < T <= max_seq):
        raise ValueError("prompt length outside the cache")
    cos, sin = ops.rotary_cos_sin(torch.arange(T), D, s.rope_theta)
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)  # (T, 1, D) against (T, heads, D)
    h = w.embed[toks].clone()
    kv_out = []
    for L in w.layers:
        r = h
        xn = ops.rms_norm(h, L.ln_in, s.eps)
        qkv = ops.linear_separate_w8(xn, unpacked_codes(L.qkv_codes, bits), L.qkv_scale, g)
        q = ops.rms_norm(qkv[:, :HD], L.q_norm, s.eps).reshape(T, NH, D)
        k = ops.rms_norm(qkv[:, HD:2 * HD], L.k_norm, s.eps).reshape(T, NH, D)
        v = qkv[:, 2 * HD:].reshape(T, NH, D)
        q, k, v = ops.clip_qkv(q, k, v, getattr(s, "clip_qkv", None))
        q, k = ops.rope_hf(q, k, cos, sin)
        if kv_cache == "fp16":
            cache = {
                "k": torch.zeros((NH, max_seq, D), dtype=torch.float16),
                "v": torch.zeros((NH, max_seq, D), dtype=torch.float16),
            }
            cache["k"][:, :T, :] = k.transpose(0, 1)
            cache["v"][:, :T, :] = v.transpose(0, 1)
        else:
            cache = {
                "kc": torch.zeros((NH, max_seq, D), dtype=torch.int8),
                "ks": torch.ones((NH, max_seq), dtype=torch.float16),
                "vc": torch.zeros((NH, max_seq, D), dtype=torch.int8),
                "vs": torch.ones((NH, max_seq), dtype=torch.float16),
            }
            for name, rows in (("k", k), ("v", v)):
                codes, scales = oq.kv_quantize_rows(rows.reshape(T * NH, D).numpy())
                cache[name + "c"][:, :T, :] = torch.from_numpy(codes).reshape(T, NH, D).transpose(0, 1)
                cache[name + "s"][:, :T] = torch.from_numpy(scales).reshape(T, NH).transpose(0, 1)
        kv_out.append(cache)
        if kv_f16 is not None:
            kv_f16.append((k.transpose(0, 1).contiguous(), v.transpose(0, 1).contiguous()))
        if kv_layers is not None and len(kv_out) >= kv_layers:
            return None, kv_out
        attn = ops.causal_attention(q, k, v).to(torch.float16).reshape(T, HD)
        h = r + ops.linear_separate_w8(attn, unpacked_codes(L.o_codes, bits), L.o_scale, g)
        r = h
        xn = ops.rms_norm(h, L.ln_post, s.eps)
        top_w, top_i = ops.route_logits(ops.linear_f16(xn, L.router), s.top_k, s.norm_topk_prob)
        h = r + ops.moe_prefill_w8(xn, unpacked_codes(L.gu_codes, bits), L.gu_scale,
                                   unpacked_codes(L.dn_codes, bits), L.dn_scale, g, top_i, top_w.to(torch.float16))
    rows = h if all_logits else h[-1:]
    hn = ops.rms_norm(rows, w.final_norm, s.eps)
    lm_f16 = getattr(w, "lm_f16", None)  # fp16 lm_head: F.linear in fp16
    logits = ops.linear_f16(hn, lm_f16) if lm_f16 is not None else ops.linear_separate_w8(hn, w.lm_codes,
                                                                                            w.lm_scale, g)
    return (logits if all_logits else logits[0]), kv_out
