"""GPU parity of the decode step's fused attention over the fp16 cache (KV-INT8
off) against the unfused operators and the CPU oracle:

* lemoq_attn_split_fused_f16 (q/k norm + RoPE + fp16 slot write + split-KV
  partials in one launch) vs lemoq_qk_norm_rope_kv_i8 (its fp16 row outputs
  written into the cache) + lemoq_attn_split_f16, both merged by
  lemoq_attn_merge.  This is the reference's KV-INT8-off glue:
  kv_direct_write of the rotated k and the v row, then the fp16 split-KV
  attention (src/lemoq/kernels/attn_decode.py:930-948,999-1008).

The fp16 cache after the launch must equal the unfused path's bit for bit (the
new row at slot pos, every other slot untouched); attention outputs must match
within the fp16 tolerance rtol 2e-2 / atol 2e-3 of each other, of the oracle's
split-KV attention over the written cache and of fp64 dense attention.  Cases
mirror the KV-INT8 kernel's: first token, wave-block and round boundaries
(a wave block here is 3 loads of 4 tokens at D 128), several split counts,
long caches, a NaN-poisoned tail that must never be read, a position outside
the cache and clip_qkv.
"""

from __future__ import annotations

import math

import pytest
import torch

from helpers import assert_close
from oracle import ops

pytestmark = pytest.mark.gpu

LOG2E = 1.4426950408889634


def _state(heads, D, S, seed):
    HD = heads * D
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn((3 * HD,), generator=g) * 2).to(torch.float16)
    qn = (torch.rand((HD,), generator=g) + 0.5).to(torch.float16)
    kn = (torch.rand((HD,), generator=g) + 0.5).to(torch.float16)
    cache = {"k": torch.randn((heads, S, D), generator=g).to(torch.float16),
             "v": torch.randn((heads, S, D), generator=g).to(torch.float16)}
    cos, sin = ops.rotary_cos_sin(torch.arange(S), D, 1e4)
    return qkv, qn, kn, cache, cos.contiguous(), sin.contiguous()


def _to(dev, cache):
    return {n: t.clone().to(dev) for n, t in cache.items()}


def _split_path(hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns, clip=math.inf):
    """Unfused: the q/k norm + RoPE launch writes the fp16 rows into the cache
    (its KV-INT8 outputs go to scratch), then the fp16 split kernel + merge."""
    c = _to(dev, cache)
    q_rot = torch.empty((heads * D,), dtype=torch.float16, device=dev)
    scratch = {"kc": torch.zeros((heads, S, D), dtype=torch.int8, device=dev),
               "ks": torch.ones((heads, S), dtype=torch.float16, device=dev)}
    scratch["vc"], scratch["vs"] = torch.zeros_like(scratch["kc"]), torch.ones_like(scratch["ks"])
    posd = torch.tensor([pos], dtype=torch.int64, device=dev)
    filled = torch.tensor([pos + 1], dtype=torch.int32, device=dev)
    m = torch.empty((heads * ns,), dtype=torch.float32, device=dev)
    l = torch.empty_like(m)
    acc = torch.empty((heads * ns * D,), dtype=torch.float32, device=dev)
    out = torch.empty((heads * D,), dtype=torch.float16, device=dev)
    P, st = hip.ptr, hip.stream_of(dev)
    qkvd, qnd, knd, cosd, sind = (t.to(dev) for t in (qkv, qn, kn, cos, sin))
    hip.call("lemoq_qk_norm_rope_kv_i8", P(qkvd), heads, D, P(qnd), P(knd), 1e-5, P(cosd), P(sind), P(posd),
             P(q_rot), P(scratch["kc"]), P(scratch["ks"]), P(scratch["vc"]), P(scratch["vs"]), S * D, S,
             P(c["k"]), P(c["v"]), S * D, None, clip, st)
    qk_scale = (1.0 / math.sqrt(D)) * LOG2E
    hip.call("lemoq_attn_split_f16", P(q_rot), P(c["k"]), P(c["v"]), S * D, P(filled), heads, D, ns, qk_scale,
             P(m), P(l), P(acc), st)
    hip.call("lemoq_attn_merge", P(m), P(l), P(acc), heads, ns, D, P(out), st)
    return out.cpu(), {n: t.cpu() for n, t in c.items()}, q_rot.cpu()


def _fused_path(hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=4, clip=math.inf):
    c = _to(dev, cache)
    posd = torch.tensor([pos], dtype=torch.int64, device=dev)
    m = torch.full((heads * ns,), float("nan"), dtype=torch.float32, device=dev)
    l = torch.full_like(m, float("nan"))
    acc = torch.full((heads * ns * D,), float("nan"), dtype=torch.float32, device=dev)
    out = torch.empty((heads * D,), dtype=torch.float16, device=dev)
    P, st = hip.ptr, hip.stream_of(dev)
    qkvd, qnd, knd, cosd, sind = (t.to(dev) for t in (qkv, qn, kn, cos, sin))
    qk_scale = (1.0 / math.sqrt(D)) * LOG2E
    hip.call("lemoq_attn_split_fused_f16", P(qkvd), heads, D, P(qnd), P(knd), 1e-5, P(cosd), P(sind), P(posd),
             P(c["k"]), P(c["v"]), S * D, S, ns, qk_scale, P(m), P(l), P(acc), clip, st)
    hip.call("lemoq_attn_merge", P(m), P(l), P(acc), heads, ns, D, P(out), st)
    return out.cpu(), {n: t.cpu() for n, t in c.items()}


CASES = [
    (16, 128, 1100, 0, 3), (16, 128, 1100, 1, 3), (16, 128, 1100, 63, 3), (16, 128, 1100, 64, 8),
    (16, 128, 1100, 1024, 3), (16, 128, 1100, 1024, 1), (16, 128, 4200, 4095, 8), (8, 64, 700, 511, 2),
    (4, 256, 300, 257, 5),
    # the decode step's 16 splits at the bench's contexts and either side of them
    (16, 128, 1100, 1024, 16), (16, 128, 1100, 1060, 16), (16, 128, 1100, 70, 16), (16, 128, 1100, 15, 16),
    (16, 128, 4200, 4096, 16), (16, 128, 4200, 4132, 16), (4, 256, 1024, 1000, 16), (8, 64, 2048, 2047, 16),
    # round boundaries: a wave block is 3 loads (12 tokens at D 128, 24 at D 64, 6 at D 256)
    # and a round of 4 waves 4x that; at 16 splits, splits of exactly one or two rounds
    # and of one round plus a token
    (16, 128, 1100, 767, 16), (16, 128, 1100, 768, 16), (16, 128, 1600, 1535, 16), (16, 128, 1600, 1536, 16),
    (8, 64, 3200, 1535, 16), (8, 64, 3200, 1536, 16), (4, 256, 1100, 383, 16), (4, 256, 1100, 384, 16),
    (4, 256, 1100, 767, 16),
]


@pytest.mark.parametrize("heads,D,S,pos,ns", CASES)
def test_fused_f16_attention_equals_split_path_and_oracle(heads, D, S, pos, ns, dev):
    from lemoq import _hip

    print("case: f16 heads=%d D=%d S=%d pos=%d ns=%d" % (heads, D, S, pos, ns), flush=True)
    qkv, qn, kn, cache, cos, sin = _state(heads, D, S, seed=pos + D + 3)
    out_s, cache_s, q_rot = _split_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=16)
    out_f, cache_f = _fused_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=ns)
    for n in ("k", "v"):
        # identical fp16 rows at slot pos, every other slot untouched
        assert torch.equal(cache_f[n].view(torch.int16), cache_s[n].view(torch.int16)), n
        keep = torch.ones(S, dtype=torch.bool)
        keep[pos] = False
        assert torch.equal(cache_f[n][:, keep].view(torch.int16), cache[n][:, keep].view(torch.int16)), n
    assert torch.isfinite(out_f).all()
    assert_close(out_f, out_s, what="fused vs split")
    # oracle: q/k norm + RoPE, the rows written as they are, attention over [0, pos]
    q = ops.rope_fused(ops.rms_norm(qkv[: heads * D], qn, 1e-5).reshape(heads, D), cos[pos], sin[pos])
    k = ops.rope_fused(ops.rms_norm(qkv[heads * D: 2 * heads * D], kn, 1e-5).reshape(heads, D), cos[pos], sin[pos])
    assert_close(q_rot, q.reshape(-1), rtol=2e-3, atol=2e-3, what="q_norm+rope")
    # GPU and CPU sum the squares in different orders: rstd may differ by an ulp
    assert_close(cache_f["k"][:, pos], k, rtol=2e-3, atol=2e-3, what="k row")
    assert torch.equal(cache_f["v"][:, pos], qkv[2 * heads * D:].reshape(heads, D))  # v as it is
    ref = ops.split_kv_oracle(q, cache_f["k"], cache_f["v"], pos + 1, num_splits=ns)
    assert_close(out_f.reshape(heads, D), ref, what="fused vs oracle")
    dense = ops.dense_attention(q, cache_f["k"], cache_f["v"], pos + 1)
    assert (out_f.reshape(heads, D).double() - dense).abs().max() < 2e-3


def test_fused_f16_attention_never_reads_beyond_pos(dev):
    """NaN-poisoned rows after pos never leak in."""
    from lemoq import _hip

    heads, D, S, pos = 16, 128, 600, 300
    qkv, qn, kn, cache, cos, sin = _state(heads, D, S, seed=11)
    clean, _ = _fused_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S)
    poisoned = {n: t.clone() for n, t in cache.items()}
    poisoned["k"][:, pos + 1:] = float("nan")
    poisoned["v"][:, pos + 1:] = float("nan")
    out, _ = _fused_path(_hip, dev, qkv, qn, kn, poisoned, cos, sin, pos, heads, D, S)
    assert torch.isfinite(out).all() and torch.equal(out, clean)


def test_fused_f16_attention_position_outside_cache_writes_nothing(dev):
    from lemoq import _hip

    heads, D, S = 4, 128, 64
    qkv, qn, kn, cache, cos, sin = _state(heads, D, S, seed=12)
    out, after = _fused_path(_hip, dev, qkv, qn, kn, cache, cos, sin, S, heads, D, S)
    for n in ("k", "v"):
        assert torch.equal(after[n].view(torch.int16), cache[n].view(torch.int16)), n
    assert (out == 0).all()


@pytest.mark.parametrize("heads,D,S,pos,ns,clip", [
    (16, 128, 1100, 0, 16, 0.8), (16, 128, 1100, 700, 16, 0.8), (8, 64, 700, 511, 4, 1.3),
    (4, 256, 300, 257, 5, 0.5),
])
def test_fused_f16_attention_clip_qkv(heads, D, S, pos, ns, clip, dev):
    """clip_qkv on the fp16 path: the same rows as the unfused launch, v clamped
    exactly as the oracle clamps it, and the bound changes the output."""
    from lemoq import _hip

    print("case: f16 clip heads=%d D=%d S=%d pos=%d ns=%d clip=%g" % (heads, D, S, pos, ns, clip), flush=True)
    qkv, qn, kn, cache, cos, sin = _state(heads, D, S, seed=pos + D + 17)
    HD = heads * D
    out_s, cache_s, _ = _split_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=16, clip=clip)
    out_f, cache_f = _fused_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=ns, clip=clip)
    for n in ("k", "v"):
        assert torch.equal(cache_f[n].view(torch.int16), cache_s[n].view(torch.int16)), n
    assert_close(out_f, out_s, what="fused vs split")
    qn_, kn_ = (ops.rms_norm(qkv[a:a + HD], w, 1e-5).reshape(heads, D) for a, w in ((0, qn), (HD, kn)))
    qc, _, vc_ = ops.clip_qkv(qn_, kn_, qkv[2 * HD:].reshape(heads, D), clip)
    assert float((vc_ != qkv[2 * HD:].reshape(heads, D)).double().mean()) > 0.05  # the bound bites
    assert torch.equal(cache_f["v"][:, pos], vc_)
    q = ops.rope_fused(qc, cos[pos], sin[pos])
    ref = ops.split_kv_oracle(q, cache_f["k"], cache_f["v"], pos + 1, num_splits=ns)
    assert_close(out_f.reshape(heads, D), ref, what="clipped fused vs oracle")
    out_n, _ = _fused_path(_hip, dev, qkv, qn, kn, cache, cos, sin, pos, heads, D, S, ns=ns)
    assert not torch.equal(out_n, out_f)
