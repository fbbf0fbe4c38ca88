"""GPU parity of the decode step's fused attention against the unfused operators
and the CPU oracle:

* lemoq_attn_split_fused_i8 (q/k norm + RoPE + KV-INT8 write + split-KV
  partials in one launch) vs lemoq_qk_norm_rope_kv_i8 + lemoq_attn_split_i8,
  both merged by lemoq_attn_merge;

The KV-INT8 bytes written must equal the unfused path's bit for bit (both are
pinned to the oracle's per-token quantiser); attention outputs must match
within the fp16 tolerance rtol 2e-2 / atol 2e-3.  Cases mirror the
reference's length boundaries (tests/test_fusion_adversarial.py:72-85,
tests/test_attn_decode.py:83-149 of LeanMoE-Quant): first token, block edges,
several split counts, long caches, a NaN-poisoned tail that must never be read.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import assert_close, randn
from oracle import ops
from oracle import quant as oq

pytestmark = pytest.mark.gpu

LOG2E = 1.4426950408889634


def _state(heads, D, S, filled, seed):
    HD = heads * D
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn((3 * HD,), generator=g) * 2).to(torch.float16)
    qn = (torch.rand((HD,), generator=g) + 0.5).to(torch.float16)
    kn = (torch.rand((HD,), generator=g) + 0.5).to(torch.float16)
    k = torch.randn((heads, S, D), generator=g).to(torch.float16)
    v = torch.randn((heads, S, D), generator=g).to(torch.float16)
    kc, ks = oq.kv_quantize_rows(k.numpy())
    vc, vs = oq.kv_quantize_rows(v.numpy())
    cache = {n: torch.from_numpy(a) for n, a in (("kc", kc), ("ks", ks), ("vc", vc), ("vs", vs))}
    cos, sin = ops.rotary_cos_sin(torch.arange(S), D, 1e4)
    return qkv, qn, kn, cache, cos.contiguous(), sin.contiguous()


def _to(dev, cache):
    return {n: t.clone().to(dev) for n, t in cache.items()}


def _split_path(hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns, clip=math.inf):
    c = _to(dev, cache)
    q_rot = torch.empty((heads * D,), dtype=torch.float16, device=dev)
    posd = torch.tensor([pos], dtype=torch.int64, device=dev)
    filled = torch.tensor([pos + 1], dtype=torch.int32, device=dev)
    m = torch.empty((heads * ns,), dtype=torch.float32, device=dev)
    l = torch.empty_like(m)
    acc = torch.empty((heads * ns * D,), dtype=torch.float32, device=dev)
    out = torch.empty((heads * D,), dtype=torch.float16, device=dev)
    P, st = hip.ptr, hip.stream_of(dev)
    qkvd, qnd, knd, cosd, sind = (t.to(dev) for t in (qkv, qn, kn, cos, sin))
    hip.call("lemoq_qk_norm_rope_kv_i8", P(qkvd), heads, D, P(qnd), P(knd), 1e-5, P(cosd), P(sind), P(posd),
             P(q_rot), P(c["kc"]), P(c["ks"]), P(c["vc"]), P(c["vs"]), S * D, S, None, None, 0, None, clip, st)
    qk_scale = (1.0 / math.sqrt(D)) * LOG2E
    hip.call("lemoq_attn_split_i8", P(q_rot), P(c["kc"]), P(c["ks"]), P(c["vc"]), P(c["vs"]), S * D, S,
             P(filled), heads, D, ns, qk_scale, P(m), P(l), P(acc), st)
    hip.call("lemoq_attn_merge", P(m), P(l), P(acc), heads, ns, D, P(out), st)
    return out.cpu(), {n: t.cpu() for n, t in c.items()}, q_rot.cpu()


def _merge(hip, dev, m, l, acc, heads, ns, D):
    out = torch.empty((heads * D,), dtype=torch.float16, device=dev)
    hip.call("lemoq_attn_merge", hip.ptr(m), hip.ptr(l), hip.ptr(acc), heads, ns, D, hip.ptr(out), hip.stream_of(dev))
    return out


def _fused_path(hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=4, raw=False, clip=math.inf):
    c = _to(dev, cache)
    posd = torch.tensor([pos], dtype=torch.int64, device=dev)
    m = torch.full((heads * ns,), float("nan"), dtype=torch.float32, device=dev)
    l = torch.full_like(m, float("nan"))
    acc = torch.full((heads * ns * D,), float("nan"), dtype=torch.float32, device=dev)
    P, st = hip.ptr, hip.stream_of(dev)
    qkvd, qnd, knd, cosd, sind = (t.to(dev) for t in (qkv, qn, kn, cos, sin))
    qk_scale = (1.0 / math.sqrt(D)) * LOG2E
    hip.call("lemoq_attn_split_fused_i8", P(qkvd), heads, D, P(qnd), P(knd), 1e-5, P(cosd), P(sind), P(posd),
             P(c["kc"]), P(c["ks"]), P(c["vc"]), P(c["vs"]), S * D, S, ns, qk_scale, P(m), P(l), P(acc), clip, st)
    if raw:
        return m, l, acc, {n: t.cpu() for n, t in c.items()}
    out = _merge(hip, dev, m, l, acc, heads, ns, D)
    return out.cpu(), {n: t.cpu() for n, t in c.items()}


@pytest.mark.parametrize("heads,D,S,pos,ns", [
    (16, 128, 1100, 0, 3), (16, 128, 1100, 1, 3), (16, 128, 1100, 63, 3), (16, 128, 1100, 64, 8),
    (16, 128, 1100, 1024, 3), (16, 128, 1100, 1024, 1), (16, 128, 4200, 4095, 8), (8, 64, 700, 511, 2),
    (4, 256, 300, 257, 5), (16, 128, 1100, 5, 8),
    # the decode step's 16 splits: splits of one token round per wave and of several
    (16, 128, 1100, 1060, 16), (16, 128, 1100, 70, 16), (16, 128, 1100, 15, 16), (16, 128, 4200, 4132, 16),
    (16, 128, 4200, 300, 16), (4, 256, 1024, 1000, 16), (8, 64, 2048, 2047, 16),
    # round boundaries of the token loop: a wave block is 3 loads (24 tokens at D 128, 48 at
    # D 64, 12 at D 256) and a round of 4 waves 4x that; splits of exactly one round, one round
    # plus a token, two rounds plus a token, and of one or two wave blocks' worth
    (16, 128, 1600, 1535, 16), (16, 128, 1600, 1536, 16), (16, 128, 3200, 3072, 16),
    (16, 128, 1100, 383, 16), (16, 128, 1100, 384, 16), (8, 64, 3200, 3071, 16), (8, 64, 3200, 3072, 16),
    (4, 256, 1100, 767, 16), (4, 256, 1100, 768, 16),
])
def test_fused_attention_equals_split_path_and_oracle(heads, D, S, pos, ns, dev):
    from lemoq import _hip

    print("case: heads=%d D=%d S=%d pos=%d ns=%d" % (heads, D, S, pos, ns), flush=True)
    qkv, qn, kn, cache, cos, sin = _state(heads, D, S, pos + 1, seed=pos + D)
    out_s, cache_s, q_rot = _split_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=16)
    out_f, cache_f = _fused_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=ns)
    for n in ("kc", "ks", "vc", "vs"):
        assert torch.equal(cache_f[n], cache_s[n]), n  # identical KV-INT8 bytes at slot pos, rest untouched
    assert torch.isfinite(out_f).all()
    assert_close(out_f, out_s, what="fused vs split")
    # oracle: q/k norm + RoPE then int8 attention over [0, pos] of the written cache
    q = ops.rope_fused(ops.rms_norm(qkv[: heads * D], qn, 1e-5).reshape(heads, D), cos[pos], sin[pos])
    # GPU and CPU sum the squares in different orders: rstd may differ by an ulp
    assert_close(q_rot, q.reshape(-1), rtol=2e-3, atol=2e-3, what="q_norm+rope")
    ref = ops.int8_attention_folded(q, cache_s["kc"], cache_s["ks"], cache_s["vc"], cache_s["vs"], pos + 1)
    assert_close(out_f.reshape(heads, D), ref, what="fused vs oracle")
    deq = ops.int8_attention_dequant(q, cache_s["kc"], cache_s["ks"], cache_s["vc"], cache_s["vs"], pos + 1)
    assert (out_f.reshape(heads, D).double() - deq).abs().max() < 2e-3


def test_fused_attention_never_reads_beyond_pos(dev):
    """NaN-poisoned slots after pos (codes cannot be NaN, scales can) never leak in."""
    from lemoq import _hip

    heads, D, S, pos = 16, 128, 600, 300
    qkv, qn, kn, cache, cos, sin = _state(heads, D, S, pos + 1, seed=11)
    clean, _ = _fused_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S)
    poisoned = {n: t.clone() for n, t in cache.items()}
    poisoned["ks"][:, pos + 1:] = float("nan")
    poisoned["vs"][:, pos + 1:] = float("nan")
    out, _ = _fused_path(_hip, dev, qkv, qn, kn, poisoned, cos, sin, pos, heads, D, S)
    assert torch.isfinite(out).all() and torch.equal(out, clean)


def test_fused_attention_position_outside_cache_writes_nothing(dev):
    from lemoq import _hip

    heads, D, S = 4, 128, 64
    qkv, qn, kn, cache, cos, sin = _state(heads, D, S, 1, seed=12)
    out, after = _fused_path(_hip, dev, qkv, qn, kn, cache, cos, sin, S, heads, D, S)
    for n in ("kc", "ks", "vc", "vs"):
        assert torch.equal(after[n], cache[n]), n
    assert (out == 0).all()




@pytest.mark.parametrize("heads,D,S,pos,ns,clip", [
    (16, 128, 1100, 0, 16, 0.8), (16, 128, 1100, 700, 16, 0.8), (8, 64, 700, 511, 4, 1.3),
    (4, 256, 300, 257, 5, 0.5), (16, 128, 1100, 300, 16, 0.0),
])
def test_fused_attention_clip_qkv(heads, D, S, pos, ns, clip, dev):
    """HF OLMoE's clip_qkv (the reference's glue clamps the normed q/k and v,
    ``src/lemoq/kernels/attn_decode.py:903-907``): the fused launch and the
    unfused q/k norm + RoPE launch write the same KV bytes, their q and v match
    the oracle's clamp, and the bound changes the output (it is not ignored)."""
    from lemoq import _hip

    print("case: clip heads=%d D=%d S=%d pos=%d ns=%d clip=%g" % (heads, D, S, pos, ns, clip), flush=True)
    qkv, qn, kn, cache, cos, sin = _state(heads, D, S, pos + 1, seed=pos + D + 7)
    HD = heads * D
    out_s, cache_s, q_rot = _split_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=16, clip=clip)
    out_f, cache_f = _fused_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=ns, clip=clip)
    for n in ("kc", "ks", "vc", "vs"):
        assert torch.equal(cache_f[n], cache_s[n]), n
    assert_close(out_f, out_s, what="fused vs split")
    qn_, kn_ = (ops.rms_norm(qkv[a:a + HD], w, 1e-5).reshape(heads, D) for a, w in ((0, qn), (HD, kn)))
    qc, kc_, vc_ = ops.clip_qkv(qn_, kn_, qkv[2 * HD:].reshape(heads, D), clip)
    clamped = float((qc != qn_).double().mean())
    assert clamped > (0.99 if clip == 0.0 else 0.05), clamped  # the bound bites
    q = ops.rope_fused(qc, cos[pos], sin[pos])
    assert_close(q_rot, q.reshape(-1), rtol=2e-3, atol=2e-3, what="clipped q_norm+rope")
    # v is stored unrotated: its codes and scale are the oracle's quantisation of the clamped row, bit for bit
    vcodes, vscale = oq.kv_quantize_rows(vc_.numpy())
    assert np.array_equal(cache_f["vc"][:, pos].numpy(), vcodes)
    assert np.array_equal(cache_f["vs"][:, pos].numpy().view(np.uint16), vscale.view(np.uint16))
    ref = ops.int8_attention_folded(q, cache_s["kc"], cache_s["ks"], cache_s["vc"], cache_s["vs"], pos + 1)
    assert_close(out_f.reshape(heads, D), ref, what="clipped fused vs oracle")
    if clip > 0.0:
        out_n, _ = _fused_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=ns)
        assert not torch.equal(out_n, out_f)
