"""Pins the CPU oracle of the reference's prefill (``oracle.olmoe.oracle_prefill``).

1. Against HF transformers ``OlmoeForCausalLM`` in float64 on the oracle's
   dequantised weights (the model the reference patches): all T positions'
   logits of one prefill pass.  The prefill keeps fp16 K/V, so it sits much
   closer to HF than the KV-INT8 decode: measured median per-position KL
   3.7e-7 .. 4.9e-7 and median max|diff| / max|logit| 0.0009 .. 0.0011 over
   three seeds; the gate is KL < 1e-5 and relative error < 0.005.  Planted
   mistakes in the oracle (RoPE sign, no causal mask, a skipped q_norm, gate and
   up swapped, routing weights dropped, experts permuted) each fail it: the
   smallest measured effect is KL 9.0e-3 / relative error 0.147.
2. ``ops.causal_attention`` row t equals ``ops.dense_attention`` (the decode
   oracle's unsplit attention, pinned separately) over keys 0..t.
3. ``ops.moe_prefill_w8`` token t equals the decode oracle's
   ``ops.grouped_moe_w8`` for that token within the rounding of the fp16
   intermediates (relative 2e-2).
4. torch's CPU ``index_add_`` on fp16 rounds after every added term (the
   per-expert accumulation the oracle relies on).
5. The prefill's KV-INT8 cache and the decode oracle's stepped cache hold the
   same tokens in the same (head, slot) layout: in layer 0, whose inputs agree,
   codes lie within one step (the two RoPE and linear roundings differ); unused
   slots keep codes 0 and scales 1.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ops
from oracle.olmoe import OracleDecoder, oracle_prefill, random_host_weights

transformers = pytest.importorskip("transformers")

from test_oracle_hf_olmoe import SHAPE, _hf_model, _stats  # noqa: E402

N_POS = 12
MED_KL = 1e-5
MED_REL = 0.005
_CACHE: dict = {}


def _case(seed):
    if seed not in _CACHE:
        hw = random_host_weights(SHAPE, seed=seed)
        toks = torch.randint(0, SHAPE.vocab, (N_POS,), generator=torch.Generator().manual_seed(seed + 100))
        with torch.no_grad():
            ref = _hf_model(hw)(toks[None]).logits[0]
        _CACHE[seed] = (hw, toks, ref)
    return _CACHE[seed]


def _passes(ref, hw, toks):
    out, _ = oracle_prefill(hw, toks, N_POS + 4, all_logits=True)
    kl, rel = _stats(ref, out.double())
    return kl < MED_KL and rel < MED_REL, (kl, rel)


@pytest.mark.parametrize("seed", [5, 6, 7])
def test_oracle_prefill_matches_hf_olmoe(seed):
    hw, toks, ref = _case(seed)
    ok, (kl, rel) = _passes(ref, hw, toks)
    assert ok, "median KL %.3e, median rel %.4f" % (kl, rel)


def test_oracle_prefill_clip_qkv_matches_hf_olmoe():
    """The prefill oracle with HF OLMoE's clip_qkv set (0.6, which clamps a large
    share of the normed q/k and of v) against HF's full forward with the same
    config, and without its clamp it fails the gate."""
    from oracle.olmoe import Shape

    shape = Shape(**{**SHAPE.__dict__, "clip_qkv": 0.6})
    hw = random_host_weights(shape, seed=9)
    toks = torch.randint(0, SHAPE.vocab, (N_POS,), generator=torch.Generator().manual_seed(109))
    with torch.no_grad():
        ref = _hf_model(hw)(toks[None]).logits[0]
    ok, (kl, rel) = _passes(ref, hw, toks)
    assert ok, "median KL %.3e, median rel %.4f" % (kl, rel)
    ok, (kl, rel) = _passes(ref, random_host_weights(SHAPE, seed=9), toks)
    assert not ok, "without the clamp the gate still passed (KL %.3e, rel %.4f)" % (kl, rel)


def _plant_rope_sign():
    orig = ops.rope_hf
    return "rope_hf", lambda q, k, c, s: orig(q, k, c, -s)


def _plant_no_mask():
    def attn(q, k, v, *, scale=None, dtype=torch.float64):
        T, dim = int(q.shape[0]), int(q.shape[-1])
        qq, kk, vv = (t.to(dtype).transpose(0, 1) for t in (q, k, v))
        sc = torch.matmul(qq, kk.transpose(1, 2)) / dim ** 0.5
        return torch.matmul(torch.softmax(sc, -1), vv).transpose(0, 1)
    return "causal_attention", attn


def _plant_moe(kind):
    orig = ops.moe_prefill_w8

    def moe(x, guc, gus, dnc, dns, g, ti, tw):
        if kind == "gate_up_swap":
            F = guc.shape[1] // 2
            guc = torch.cat([guc[:, F:], guc[:, :F]], 1)
            gus = torch.cat([gus[:, F:], gus[:, :F]], 1)
        elif kind == "unweighted":
            tw = torch.ones_like(tw)
        elif kind == "experts_permuted":
            ti = (ti + 1) % guc.shape[0]
        return orig(x, guc, gus, dnc, dns, g, ti, tw)
    return "moe_prefill_w8", moe


def _plant_skip_q_norm(hw):
    targets = [L.q_norm for L in hw.layers]
    orig = ops.rms_norm
    return "rms_norm", lambda x, w, eps: x if any(w is t for t in targets) else orig(x, w, eps)


PLANTED = {
    "rope_sign": lambda hw: _plant_rope_sign(),
    "no_causal_mask": lambda hw: _plant_no_mask(),
    "q_norm_skipped": _plant_skip_q_norm,
    "gate_up_swapped": lambda hw: _plant_moe("gate_up_swap"),
    "route_weights_dropped": lambda hw: _plant_moe("unweighted"),
    "experts_permuted": lambda hw: _plant_moe("experts_permuted"),
}


@pytest.mark.parametrize("mistake", sorted(PLANTED))
def test_planted_prefill_mistake_fails_the_hf_gate(mistake, monkeypatch):
    hw, toks, ref = _case(5)
    name, fn = PLANTED[mistake](hw)
    monkeypatch.setattr(ops, name, fn)
    ok, (kl, rel) = _passes(ref, hw, toks)
    assert not ok, "%s went unnoticed: median KL %.3e, median rel %.4f" % (mistake, kl, rel)


def test_causal_attention_rows_equal_dense_attention():
    g = torch.Generator().manual_seed(3)
    T, NH, D = 37, 3, 64
    q, k, v = (torch.randn((T, NH, D), generator=g).to(torch.float16) for _ in range(3))
    out = ops.causal_attention(q, k, v)
    kk, vv = k.transpose(0, 1), v.transpose(0, 1)
    for t in range(T):
        ref = ops.dense_attention(q[t], kk, vv, t + 1)
        assert torch.allclose(out[t], ref, rtol=1e-12, atol=1e-12), t


def test_moe_prefill_matches_the_decode_moe_per_token():
    hw = random_host_weights(SHAPE, seed=9)
    L = hw.layers[0]
    s = SHAPE
    g = torch.Generator().manual_seed(10)
    T = 20
    x = (torch.randn((T, s.hidden), generator=g)).to(torch.float16)
    top_w, top_i = ops.route_logits(ops.linear_f16(x, L.router), s.top_k, s.norm_topk_prob)
    out = ops.moe_prefill_w8(x, L.gu_codes, L.gu_scale, L.dn_codes, L.dn_scale, s.group_size, top_i,
                             top_w.to(torch.float16))
    for t in range(T):
        ref, _ = ops.grouped_moe_w8(x[t], L.gu_codes, L.gu_scale, L.dn_codes, L.dn_scale, s.group_size,
                                    top_i[t], top_w[t].to(torch.float16))
        err = float((out[t].double() - ref.double()).abs().max())
        assert err <= 2e-2 * float(ref.double().abs().max()) + 1e-3, (t, err)


def test_fp16_index_add_rounds_after_every_term():
    out = torch.zeros(2, dtype=torch.float16)
    idx = torch.tensor([0])
    out.index_add_(0, idx, torch.tensor([2048.0], dtype=torch.float16))
    out.index_add_(0, idx, torch.tensor([1.0], dtype=torch.float16))
    out.index_add_(0, idx, torch.tensor([1.0], dtype=torch.float16))
    assert float(out[0]) == 2048.0  # fp32 accumulation would give 2050


def test_prefill_kv_cache_layout_matches_the_stepped_cache():
    hw, toks, _ = _case(6)
    _, kv = oracle_prefill(hw, toks, N_POS + 4)
    o = OracleDecoder(hw, N_POS + 4)
    for p, t in enumerate(toks):
        o.step(int(t), p)
    # layer 0 sees the same inputs in both (deeper layers inherit the rounding differences)
    for name in ("kc", "vc"):
        a, b = kv[0][name][:, :N_POS].int(), o.kv[0][name][:, :N_POS].int()
        assert int((a - b).abs().max()) <= 1 and float((a == b).double().mean()) > 0.95, name
    for li in range(SHAPE.layers):
        assert torch.equal(kv[li]["kc"][:, N_POS:], torch.zeros_like(kv[li]["kc"][:, N_POS:]))
        assert torch.equal(kv[li]["ks"][:, N_POS:], torch.ones_like(kv[li]["ks"][:, N_POS:]))


def test_separate_arm_weight_is_one_rounding_of_the_exact_product():
    """code (8 bits) x fp16 scale (11 significant bits) fits fp32 exactly, so the reference's
    ``dequantized_weight(dtype=fp16)`` (fp32 product, then ``.to(fp16)``) rounds once."""
    g = torch.Generator().manual_seed(21)
    codes = torch.randint(-128, 128, (64, 256), generator=g, dtype=torch.int8)
    scale = (torch.rand((64, 2), generator=g) * 1e-2 + 1e-5).to(torch.float16)
    w32 = ops.dequant_w8(codes, scale, 128)
    w64 = codes.double() * scale.double().repeat_interleave(128, 1)
    assert torch.equal(w32.double(), w64)
    assert torch.equal(ops.dequant_weight_f16(codes, scale, 128), w64.to(torch.float16))
    # and the separate arm differs from the fused arm's single fp32 rounding of the sum
    x = torch.randn((3, 256), generator=g).to(torch.float16)
    sep = ops.linear_separate_w8(x, codes, scale, 128).double()
    ref = x.double() @ w64.t()
    assert float((sep - ref).abs().max()) < 2e-2 * float(ref.abs().max())


def test_prefill_kv_rows_hook_matches_the_cache_and_stops_early():
    """``oracle_prefill(kv_f16=...)`` hands out the fp16 rows its cache bytes were
    quantised from (the GPU parity tests compare the GPU's rows and bytes with
    them), and ``kv_layers`` stops after that many layers with the same bytes."""
    import numpy as np

    from oracle import quant as oq

    w = random_host_weights(SHAPE, seed=5)
    toks = [3, 17, 17, 42, 9, 3, 60]
    rows = []
    _, kv = oracle_prefill(w, toks, 12, kv_f16=rows)
    assert len(rows) == SHAPE.layers
    T = len(toks)
    for li, (k16, v16) in enumerate(rows):
        assert k16.shape == (SHAPE.heads, T, SHAPE.head_dim) and k16.dtype == torch.float16
        for name, r in (("k", k16), ("v", v16)):
            c, s = oq.kv_quantize_rows(r.reshape(-1, SHAPE.head_dim).numpy())
            assert np.array_equal(kv[li][name + "c"][:, :T].reshape(-1, SHAPE.head_dim).numpy(), c)
            assert np.array_equal(kv[li][name + "s"][:, :T].reshape(-1).numpy().view(np.uint16), s.view(np.uint16))
    rows1 = []
    lg, kv1 = oracle_prefill(w, toks, 12, kv_f16=rows1, kv_layers=1)
    assert lg is None and len(kv1) == 1 and len(rows1) == 1
    assert all(torch.equal(kv1[0][n], kv[0][n]) for n in ("kc", "ks", "vc", "vs"))
    assert torch.equal(rows1[0][0], rows[0][0]) and torch.equal(rows1[0][1], rows[0][1])


def test_prefill_fp16_cache_holds_the_rows_of_the_int8_cache():
    """``oracle_prefill(kv_cache="fp16")`` keeps the fp16 k/v rows that the KV-INT8
    prefill quantises (``kv_f16``) at the same slots, zeros past the prompt, and its
    last logits match HF under the same gate; the fp16-cache decoder stepped over the
    prompt writes layer 0's rows at the same slots: within 0.5% of the rows' largest
    value (measured 0.06-0.13%: the fused against the separate linear arm and RoPE
    rounding), while rows one slot apart differ by over 100%."""
    hw, toks, ref = _case(6)
    rows: list = []
    _, kv8 = oracle_prefill(hw, toks, N_POS + 4, kv_f16=rows)
    logits, kv = oracle_prefill(hw, toks, N_POS + 4, kv_cache="fp16", all_logits=True)
    for li in range(SHAPE.layers):
        assert torch.equal(kv[li]["k"][:, :N_POS], rows[li][0])
        assert torch.equal(kv[li]["v"][:, :N_POS], rows[li][1])
        assert not kv[li]["k"][:, N_POS:].any() and not kv[li]["v"][:, N_POS:].any()
    kl, rel = _stats(ref, logits.double())
    assert kl < MED_KL and rel < MED_REL, (kl, rel)
    o = OracleDecoder(hw, N_POS + 4, kv_cache="fp16")
    for p, t in enumerate(toks):
        o.step(int(t), p)
    for name in ("k", "v"):
        a, b = kv[0][name][:, :N_POS].double(), o.kv[0][name][:, :N_POS].double()
        top = float(a.abs().max())
        assert float((a - b).abs().max()) <= 5e-3 * top, name
        assert float((a[:, 1:] - b[:, :-1]).abs().max()) > 0.5 * top, name


@pytest.mark.parametrize("seed", [5, 6])
def test_oracle_prefill_w4_fp16_lm_head_matches_hf_olmoe(seed):
    """The w4a16 cell's prefill (4-bit codes unpacked before the separate arm, the
    fp16 lm_head as an fp16 F.linear) against HF OlmoeForCausalLM in fp64 loaded
    with the same dequantised weights and fp16 lm_head, with the prefill gate; its
    KV-INT8 rows match the stepped 4-bit decoder's at the same slots."""
    hw = random_host_weights(SHAPE, seed=seed, bits=4, lm_head="fp16")
    toks = torch.randint(0, SHAPE.vocab, (N_POS,), generator=torch.Generator().manual_seed(seed + 400))
    with torch.no_grad():
        ref = _hf_model(hw)(toks[None]).logits[0]
    ok, (kl, rel) = _passes(ref, hw, toks)
    assert ok, "median KL %.3e, median rel %.4f" % (kl, rel)
    _, kv = oracle_prefill(hw, toks, N_POS + 4)
    dec = OracleDecoder(hw, N_POS + 4)
    for p, t in enumerate(toks.tolist()):
        dec.step(int(t), p)
    diff = (kv[0]["kc"][:, :N_POS].int() - dec.kv[0]["kc"][:, :N_POS].int()).abs().max()
    assert int(diff) <= 1  # layer 0: the same rows up to the separate / fused rounding (one code)
