"""Pins the structure of the CPU oracle's decode step (``oracle.olmoe.OracleDecoder``)
against an independent implementation: the installed HF transformers
``OlmoeForCausalLM`` in float64, loaded with the oracle's dequantised weights.

The reference's canonical cell is HF OLMoE with its modules patched
(``src/lemoq/kernels/attn_decode.py:836-1017``, ``moe_static.py:438-534``,
``moe_grouped_quant.py:562-601``, ``rmsnorm.py:205-242``), so the HF model
is the ground truth for everything the oracle composes:
- norm placement, q/k norm over heads * D;
- the rotate_half sign;
- residuals, softmax top-k routing and its weights;
- gate/up order and the SiLU.

The oracle keeps the cell's fp16 rounding points and its KV-INT8 cache; HF
keeps neither.  So the gate is statistical over 12 teacher-forced positions:
median per-position KL(HF || oracle) < 2e-4 and median per-position
max|diff| / max|logit| < 0.025.  Measured clean over five seeds: median KL
2.4e-5 .. 3.5e-5, median relative error 0.008.  A single near-tie expert flip
can move one position to KL 2.6e-3, which the median tolerates.

Every planted mistake below fails the gate.  The mistakes are planted in the
oracle on the CPU: a flipped or dropped RoPE, a skipped q/k/input/
post-attention norm, routing weights paired with the wrong experts, forced
top-k renormalisation, gate and up swapped, routing weights dropped.  Their
smallest measured effect is median KL 1.5e-3 and median relative error
0.069, at least 2.8x beyond the gate.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ops
from oracle.olmoe import OracleDecoder, Shape, lm_head_weight, random_host_weights, unpacked_codes

transformers = pytest.importorskip("transformers")

SHAPE = Shape(hidden=256, heads=2, head_dim=128, layers=2, num_experts=8, top_k=2, ffn=128, vocab=512,
              init_std=0.05)
N_POS = 12
MED_KL = 2e-4
MED_REL = 0.025


def _hf_model(hw):
    from transformers import OlmoeConfig, OlmoeForCausalLM
    from transformers.utils import logging as hf_logging

    hf_logging.set_verbosity_error()
    s = hw.shape
    cfg = OlmoeConfig(clip_qkv=s.clip_qkv, vocab_size=s.vocab, hidden_size=s.hidden, intermediate_size=s.ffn,
                      num_hidden_layers=s.layers, num_attention_heads=s.heads, num_key_value_heads=s.heads,
                      num_experts=s.num_experts, num_experts_per_tok=s.top_k, norm_topk_prob=s.norm_topk_prob,
                      rms_norm_eps=s.eps, rope_theta=s.rope_theta, max_position_embeddings=64,
                      tie_word_embeddings=False, eos_token_id=None, pad_token_id=None, bos_token_id=None,
                      experts_implementation="eager", attn_implementation="eager")
    m = OlmoeForCausalLM(cfg).double().eval()
    g, HD, E = s.group_size, s.heads * s.head_dim, s.num_experts

    def dq(codes, scale):
        return ops.dequant_w8(unpacked_codes(codes, getattr(hw, "bits", 8)), scale, g).double()

    with torch.no_grad():
        m.model.embed_tokens.weight.copy_(hw.embed.double())
        for layer, L in zip(m.model.layers, hw.layers):
            at = layer.self_attn
            w = dq(L.qkv_codes, L.qkv_scale)
            at.q_proj.weight.copy_(w[:HD])
            at.k_proj.weight.copy_(w[HD:2 * HD])
            at.v_proj.weight.copy_(w[2 * HD:])
            at.o_proj.weight.copy_(dq(L.o_codes, L.o_scale))
            at.q_norm.weight.copy_(L.q_norm.double())
            at.k_norm.weight.copy_(L.k_norm.double())
            layer.input_layernorm.weight.copy_(L.ln_in.double())
            layer.post_attention_layernorm.weight.copy_(L.ln_post.double())
            layer.mlp.gate.weight.copy_(L.router.double())
            layer.mlp.experts.gate_up_proj.copy_(torch.stack([dq(L.gu_codes[e], L.gu_scale[e]) for e in range(E)]))
            layer.mlp.experts.down_proj.copy_(torch.stack([dq(L.dn_codes[e], L.dn_scale[e]) for e in range(E)]))
        m.model.norm.weight.copy_(hw.final_norm.double())
        m.lm_head.weight.copy_(lm_head_weight(hw).double())
    return m


_CACHE: dict = {}


def _case(seed):
    if seed not in _CACHE:
        hw = random_host_weights(SHAPE, seed=seed)
        toks = torch.randint(0, SHAPE.vocab, (N_POS,), generator=torch.Generator().manual_seed(seed + 100))
        with torch.no_grad():
            ref = _hf_model(hw)(toks[None]).logits[0]
        _CACHE[seed] = (hw, toks, ref)
    return _CACHE[seed]


def _oracle_logits(hw, toks):
    o = OracleDecoder(hw, max_seq=N_POS + 4)
    return torch.stack([o.step(int(t), p).double() for p, t in enumerate(toks)])


def _stats(ref, out):
    p, q = torch.log_softmax(ref, -1), torch.log_softmax(out, -1)
    kl = (p.exp() * (p - q)).sum(-1)
    rel = (out - ref).abs().max(-1).values / ref.abs().max()
    return float(kl.median()), float(rel.median())


def _passes(ref, out):
    kl, rel = _stats(ref, out)
    return kl < MED_KL and rel < MED_REL, (kl, rel)


# clip_qkv small enough to clamp a large share of the normed q/k and of v
SHAPE_CLIP = Shape(**{**SHAPE.__dict__, "clip_qkv": 0.6})


def test_oracle_clip_qkv_matches_hf_olmoe():
    """HF OLMoE's clip_qkv (after q_norm/k_norm, before RoPE, and on v; the
    reference's glue at src/lemoq/kernels/attn_decode.py:903-907): the oracle
    with the clamp passes the same gate against HF with ``clip_qkv`` set; the
    oracle without it, or clamping before the norms, fails it."""
    hw = random_host_weights(SHAPE_CLIP, seed=8)
    toks = torch.randint(0, SHAPE.vocab, (N_POS,), generator=torch.Generator().manual_seed(108))
    with torch.no_grad():
        ref = _hf_model(hw)(toks[None]).logits[0]
    # the clamp must bite: a large share of the oracle's first-layer q values lie beyond it
    L = hw.layers[0]
    xn = ops.rms_norm(hw.embed[toks], L.ln_in, SHAPE.eps)
    q = ops.rms_norm(ops.linear_separate_w8(xn, L.qkv_codes, L.qkv_scale, SHAPE.group_size)[:, :256], L.q_norm,
                     SHAPE.eps)
    assert float((q.float().abs() > 0.6).float().mean()) > 0.2
    ok, (kl, rel) = _passes(ref, _oracle_logits(hw, toks))
    assert ok, "with the clamp: median KL %.3e, median rel %.4f" % (kl, rel)
    hw_none = random_host_weights(SHAPE, seed=8)  # same tensors, no clamp in the oracle
    ok, (kl, rel) = _passes(ref, _oracle_logits(hw_none, toks))
    assert not ok, "without the clamp the gate still passed (KL %.3e, rel %.4f)" % (kl, rel)
    orig_norm, orig_clip = ops.rms_norm, ops.clip_qkv
    targets = [L.q_norm for L in hw.layers] + [L.k_norm for L in hw.layers]
    try:
        # planted: q and k clamped before q_norm / k_norm instead of after (v as before)
        def norm_of_clipped(x, w, eps):
            if any(w is t for t in targets):
                x = x.clamp(min=-0.6, max=0.6)
            return orig_norm(x, w, eps)

        ops.rms_norm = norm_of_clipped
        ops.clip_qkv = lambda q, k, v, c: (q, k, v.clamp(min=-c, max=c))
        ok, (kl, rel) = _passes(ref, _oracle_logits(hw, toks))
    finally:
        ops.rms_norm, ops.clip_qkv = orig_norm, orig_clip
    assert not ok, "clamping before the norms still passed (KL %.3e, rel %.4f)" % (kl, rel)


@pytest.mark.parametrize("seed", [5, 6, 7])
def test_oracle_decoder_matches_hf_olmoe(seed):
    hw, toks, ref = _case(seed)
    ok, (kl, rel) = _passes(ref, _oracle_logits(hw, toks))
    assert ok, "median KL %.3e, median rel %.4f" % (kl, rel)


def _skip_norm(which):
    def plant(hw):
        targets = [getattr(L, which) for L in hw.layers]
        orig = ops.rms_norm
        return "rms_norm", lambda x, w, eps: x if any(w is t for t in targets) else orig(x, w, eps)
    return plant


def _plant_rope(kind):
    def plant(hw):
        orig = ops.rope_fused
        if kind == "sign":
            return "rope_fused", lambda x, c, s: orig(x, c, -s)
        return "rope_fused", lambda x, c, s: x
    return plant


def _plant_route(kind):
    def plant(hw):
        orig = ops.route

        def route(x, w, k, norm):
            lg, tw, ti = orig(x, w, k, True if kind == "renorm" else norm)
            return (lg, tw, ti.flip(-1)) if kind == "pairing" else (lg, tw, ti)
        return "route", route
    return plant


def _plant_moe(kind):
    def plant(hw):
        orig = ops.grouped_moe_w8

        def moe(x, guc, gus, dnc, dns, g, ids, tw):
            if kind == "gate_up_swap":
                F = guc.shape[1] // 2
                guc = torch.cat([guc[:, F:], guc[:, :F]], 1)
                gus = torch.cat([gus[:, F:], gus[:, :F]], 1)
            if kind == "unweighted":
                tw = torch.ones_like(tw)
            return orig(x, guc, gus, dnc, dns, g, ids, tw)
        return "grouped_moe_w8", moe
    return plant


PLANTED = {
    "rope_sign": _plant_rope("sign"),
    "rope_dropped": _plant_rope("none"),
    "q_norm_skipped": _skip_norm("q_norm"),
    "k_norm_skipped": _skip_norm("k_norm"),
    "input_norm_skipped": _skip_norm("ln_in"),
    "post_attn_norm_skipped": _skip_norm("ln_post"),
    "route_weights_mispaired": _plant_route("pairing"),
    "route_forced_renorm": _plant_route("renorm"),
    "gate_up_swapped": _plant_moe("gate_up_swap"),
    "route_weights_dropped": _plant_moe("unweighted"),
}


@pytest.mark.parametrize("mistake", sorted(PLANTED))
def test_planted_oracle_mistake_fails_the_hf_gate(mistake, monkeypatch):
    hw, toks, ref = _case(5)
    name, fn = PLANTED[mistake](hw)
    monkeypatch.setattr(ops, name, fn)
    ok, (kl, rel) = _passes(ref, _oracle_logits(hw, toks))
    assert not ok, "%s went unnoticed: median KL %.3e, median rel %.4f" % (mistake, kl, rel)


# ---------------------------------------------------------------------------
# The fp16 cache (KV-INT8 off): the new k (normed, rotated) and v rows are
# written as they are and the fp16 split-KV attention reads [0, pos + 1)
# (src/lemoq/kernels/attn_decode.py:930-948,999-1008).  HF keeps its cache in
# the model's dtype, so the same gate holds, and without the KV-INT8 rounding
# the oracle sits closer to HF than the KV-INT8 oracle does.
def _oracle_logits_fp16(hw, toks):
    o = OracleDecoder(hw, max_seq=N_POS + 4, kv_cache="fp16")
    return torch.stack([o.step(int(t), p).double() for p, t in enumerate(toks)])


@pytest.mark.parametrize("seed", [5, 6, 7])
def test_oracle_fp16_cache_decoder_matches_hf_olmoe(seed):
    hw, toks, ref = _case(seed)
    ok, (kl, rel) = _passes(ref, _oracle_logits_fp16(hw, toks))
    assert ok, "median KL %.3e, median rel %.4f" % (kl, rel)
    kl8, _ = _stats(ref, _oracle_logits(hw, toks))
    assert kl <= kl8, "fp16 cache KL %.3e above the KV-INT8 cache's %.3e" % (kl, kl8)


def _plant_kv_fp16(kind):
    def plant(hw):
        orig = ops.split_kv_oracle

        def attend(q, k, v, filled, **kw):
            if kind == "new_token_dropped":  # attends over [0, pos) only
                return orig(q, k, v, filled - 1, **kw) if filled > 1 else orig(q, k, v, filled, **kw)
            return orig(q, v, k, filled, **kw)  # k and v exchanged
        return "split_kv_oracle", attend
    return plant


@pytest.mark.parametrize("mistake", ["new_token_dropped", "k_v_swapped"])
def test_planted_fp16_cache_mistake_fails_the_hf_gate(mistake, monkeypatch):
    hw, toks, ref = _case(5)
    name, fn = _plant_kv_fp16(mistake)(hw)
    monkeypatch.setattr(ops, name, fn)
    ok, (kl, rel) = _passes(ref, _oracle_logits_fp16(hw, toks))
    assert not ok, "%s went unnoticed: median KL %.3e, median rel %.4f" % (mistake, kl, rel)


# ---------------------------------------------------------------------------
# The reference's w4a16 cell: attention and experts as 4-bit symmetric codes
# (packed two per byte), the lm_head in fp16 (benchmarks/runner.py:393-412,
# 451-482).  HF is loaded with the same unpacked, dequantised weights and the
# fp16 lm_head, so the same gate applies; a planted nibble-order mistake in the
# unpacking (high nibble first) fails it.
@pytest.mark.parametrize("seed", [5, 6])
def test_oracle_w4_fp16_lm_head_matches_hf_olmoe(seed):
    hw = random_host_weights(SHAPE, seed=seed, bits=4, lm_head="fp16")
    assert hw.layers[0].qkv_codes.shape[1] == SHAPE.hidden // 2 and hw.lm_codes is None
    toks = torch.randint(0, SHAPE.vocab, (N_POS,), generator=torch.Generator().manual_seed(seed + 300))
    with torch.no_grad():
        ref = _hf_model(hw)(toks[None]).logits[0]
    ok, (kl, rel) = _passes(ref, _oracle_logits(hw, toks))
    assert ok, "median KL %.3e, median rel %.4f" % (kl, rel)


def test_planted_nibble_order_fails_the_w4_hf_gate(monkeypatch):
    import oracle.olmoe as om

    hw = random_host_weights(SHAPE, seed=5, bits=4, lm_head="fp16")
    toks = torch.randint(0, SHAPE.vocab, (N_POS,), generator=torch.Generator().manual_seed(305))
    with torch.no_grad():
        ref = _hf_model(hw)(toks[None]).logits[0]
    orig = om.unpacked_codes

    def swapped(codes, bits):
        u = orig(codes, bits)
        if int(bits) != 4:
            return u
        return u.reshape(*u.shape[:-1], -1, 2).flip(-1).reshape(u.shape)  # high nibble first

    monkeypatch.setattr(om, "unpacked_codes", swapped)
    ok, (kl, rel) = _passes(ref, _oracle_logits(hw, toks))
    assert not ok, "a swapped nibble order went unnoticed: median KL %.3e, median rel %.4f" % (kl, rel)
