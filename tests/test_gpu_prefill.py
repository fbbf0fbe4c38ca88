"""GPU parity of the batched prefill against the CPU oracle of the reference's prefill.

Per kernel:
- ``lemoq_gather_rows``: exact rows, zero rows for ids outside the table.
- ``lemoq_qk_norm_rope_kv_i8_rows``: q and k against q_norm/k_norm + HF
  ``apply_rotary_pos_emb`` (``ops.rope_hf``) within 1e-3, and equal to it in
  at least 97% of the elements (the single-rounding RoPE of the decode step
  matches clearly less often, so the test tells the two roundings apart); the
  KV-INT8 rows are bit-exactly the oracle's quantisation of the kernel's fp16
  k and v; slots past the prompt stay untouched.
- ``lemoq_attn_prefill_f16``: causal attention against fp64
  (``ops.causal_attention``), rtol 2e-2 / atol 2e-3;
  T from 1 to 2048, head_dim 64/128/256.
- MoE prefill: the sort is checked exactly (stable expert order, offsets,
  tiles); the block output (with residual) against ``ops.moe_prefill_w8``
  (the reference's per-expert loop) fed with the GPU's own routing, at the
  same tolerance, including skewed routing (experts with several tiles)
  and the OLMoE shape.
- Whole prefill (``DecodeSession.prefill()``): the last position's logits
  against ``oracle_prefill`` (KL < 0.01, max|diff| <= 2% of max|logit|), the
  seed token equal unless the oracle's top-2 margin is within the measured
  difference, the KV-INT8 cache of layer 0 within one code of the oracle's,
  then greedy decode steps from the prefilled cache against the CPU decode
  oracle on the GPU's own cache.  Tiny shape and OLMoE-1B-7B shape.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import assert_close, kv_rows_vs_oracle, randn
from oracle import ops
from oracle import quant as oq
from oracle.olmoe import OracleDecoder, oracle_prefill

pytestmark = pytest.mark.gpu

LOG2E = 1.4426950408889634


def test_gather_rows(dev):
    from lemoq import _hip

    print("case: gather_rows", flush=True)
    table = randn(50, 264, seed=1).to(torch.float16)
    ids = torch.tensor([3, 0, 49, -1, 50, 7, 7], dtype=torch.int64)
    td, idd = table.to(dev), ids.to(dev)
    out = torch.full((7, 264), 5.0, dtype=torch.float16, device=dev)
    _hip.call("lemoq_gather_rows", _hip.ptr(td), 50, 264, _hip.ptr(idd), 7, _hip.ptr(out), _hip.stream_of(dev))
    torch.cuda.synchronize()
    got = out.cpu()
    for r, i in enumerate(ids.tolist()):
        ref = table[i] if 0 <= i < 50 else torch.zeros(264, dtype=torch.float16)
        assert torch.equal(got[r], ref), r


@pytest.mark.parametrize("D,clip", [(64, math.inf), (128, math.inf), (128, 0.7)])
def test_qk_norm_rope_rows_vs_oracle(D, clip, dev):
    """With ``clip`` finite, HF OLMoE's clip_qkv clamps the normed q/k and v
    before RoPE (``src/lemoq/kernels/attn_decode.py:903-907``)."""
    from lemoq import _hip

    print("case: qk_norm_rope rows D=%d clip=%g" % (D, clip), flush=True)
    T, NH, S = 37, 4, 50
    HD = NH * D
    qkv = randn(T, 3 * HD, seed=D).to(torch.float16)
    qn = (torch.rand(HD, generator=torch.Generator().manual_seed(2)) + 0.5).to(torch.float16)
    kn = (torch.rand(HD, generator=torch.Generator().manual_seed(3)) + 0.5).to(torch.float16)
    cos, sin = ops.rotary_cos_sin(torch.arange(S), D, 10000.0)
    i8 = dict(dtype=torch.int8, device=dev)
    f16 = dict(dtype=torch.float16, device=dev)
    kc, vc = torch.zeros((NH, S, D), **i8), torch.zeros((NH, S, D), **i8)
    ks, vs = torch.ones((NH, S), **f16), torch.ones((NH, S), **f16)
    kf, vf = torch.zeros((NH, S, D), **f16), torch.zeros((NH, S, D), **f16)
    q_out = torch.empty((T, HD), **f16)
    qkv_d, qn_d, kn_d, cos_d, sin_d = (t.to(dev) for t in (qkv, qn, kn, cos, sin))
    P = _hip.ptr
    _hip.call("lemoq_qk_norm_rope_kv_i8_rows", P(qkv_d), T, NH, D, P(qn_d), P(kn_d), 1e-5, P(cos_d), P(sin_d), 0,
              P(q_out), P(kc), P(ks), P(vc), P(vs), S * D, S, P(kf), P(vf), S * D, clip, _hip.stream_of(dev))
    torch.cuda.synchronize()
    q = ops.rms_norm(qkv[:, :HD], qn, 1e-5).reshape(T, NH, D)
    k = ops.rms_norm(qkv[:, HD:2 * HD], kn, 1e-5).reshape(T, NH, D)
    v = qkv[:, 2 * HD:].reshape(T, NH, D)
    if math.isfinite(clip):
        q0 = q
        q, k, v = ops.clip_qkv(q, k, v, clip)
        assert float((q != q0).double().mean()) > 0.2  # the bound bites
    c, s_ = cos[:T].unsqueeze(1), sin[:T].unsqueeze(1)
    q_ref, k_ref = ops.rope_hf(q, k, c, s_)
    q_got = q_out.cpu().reshape(T, NH, D)
    k_got = kf[:, :T].cpu().transpose(0, 1)
    assert_close(q_got, q_ref, rtol=1e-3, atol=1e-3, what="q")
    assert_close(k_got, k_ref, rtol=1e-3, atol=1e-3, what="k")
    exact = float((q_got == q_ref).double().mean())
    fused_q = torch.stack([ops.rope_fused(q[t], cos[t], sin[t]) for t in range(T)])
    exact_fused = float((q_got == fused_q).double().mean())
    print("q exact vs HF rope %.4f, vs single-rounding rope %.4f" % (exact, exact_fused))
    assert exact >= 0.97 and exact > exact_fused
    assert torch.equal(vf[:, :T].cpu().transpose(0, 1), v)
    for codes, scales, rows in ((kc, ks, k_got), (vc, vs, v)):
        rc, rs = oq.kv_quantize_rows(rows.reshape(T * NH, D).numpy())
        assert np.array_equal(codes[:, :T].cpu().transpose(0, 1).reshape(T * NH, D).numpy(), rc)
        assert np.array_equal(scales[:, :T].cpu().transpose(0, 1).reshape(-1).numpy().view(np.uint16),
                              rs.view(np.uint16))
        assert (codes[:, T:] == 0).all() and (scales[:, T:] == 1).all()


# (T, head_dim, heads).  Fewer than 512 blocks of 128 queries take the key-split
# kernel (64 queries per block, each tile's keys split between wave pairs); the
# (777, 128, 80), (300, 64, 200) and (2048, 128, 32) cases take the unsplit one
# on the paired grid (an even number of heads; 2048 x 32 heads is 512 blocks,
# the whole grid resident as at ctx 4096 with 16 heads), (1024, 128, 65) on the
# two-dimensional grid (an odd number of heads).
ATTN_CASES = [(1, 128, 3), (7, 64, 3), (64, 128, 3), (129, 128, 3), (300, 256, 3), (2048, 128, 2),
              (777, 128, 80), (300, 64, 200), (2048, 128, 32), (1024, 128, 65)]


@pytest.mark.parametrize("T,D,NH", ATTN_CASES, ids=["T%d-D%d-H%d" % c for c in ATTN_CASES])
def test_attn_prefill_vs_fp64(T, D, NH, dev):
    from lemoq import _hip

    print("case: attn_prefill T=%d D=%d heads=%d" % (T, D, NH), flush=True)
    S = T + 5
    g = torch.Generator().manual_seed(T * 7 + D)
    q = torch.randn((T, NH, D), generator=g).to(torch.float16)
    k = torch.randn((T, NH, D), generator=g).to(torch.float16)
    v = torch.randn((T, NH, D), generator=g).to(torch.float16)
    kd = torch.zeros((NH, S, D), dtype=torch.float16)
    vd = torch.zeros((NH, S, D), dtype=torch.float16)
    kd[:, :T], vd[:, :T] = k.transpose(0, 1), v.transpose(0, 1)
    qd, kd, vd = q.reshape(T, NH * D).to(dev), kd.to(dev), vd.to(dev)
    out = torch.empty((T, NH * D), dtype=torch.float16, device=dev)
    qk_scale = (1.0 / math.sqrt(D)) * LOG2E
    _hip.call("lemoq_attn_prefill_f16", _hip.ptr(qd), NH * D, _hip.ptr(kd), _hip.ptr(vd), S * D, T, NH, D,
              qk_scale, _hip.ptr(out), NH * D, _hip.stream_of(dev))
    torch.cuda.synchronize()
    ref = ops.causal_attention(q, k, v)
    assert_close(out.cpu().reshape(T, NH, D), ref, what="attn_prefill T=%d D=%d" % (T, D))


def _moe_case(T, H, F, E, K, seed, dev, *, skew=False):
    """Random x, router and w8 expert weights (host tensors)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((T, H), generator=g)
    router = torch.randn((E, H), generator=g) * 0.02
    if skew:  # a shared offset in x lifts experts 0..K for every token: several tiles per expert
        x = x + 0.5
        router[: K + 1] += 0.02
    x, router = x.to(torch.float16), router.to(torch.float16)
    # random codes and per-group scales (weights of std ~0.02), as RTN would store them
    gu_c = torch.randint(-127, 128, (E, 2 * F, H), generator=g, dtype=torch.int8)
    dn_c = torch.randint(-127, 128, (E, H, F), generator=g, dtype=torch.int8)
    gu_s = ((torch.rand((E, 2 * F, H // 128), generator=g) + 0.5) * (0.035 / 127)).to(torch.float16)
    dn_s = ((torch.rand((E, H, F // 128), generator=g) + 0.5) * (0.035 / 127)).to(torch.float16)
    return x, router, gu_c, gu_s, dn_c, dn_s


MOE_CASES = [(1, 256, 128, 8, 2, False), (5, 256, 128, 8, 2, False), (100, 2048, 1024, 64, 8, False),
             (600, 512, 256, 16, 4, True), (300, 256, 128, 8, 8, False)]


@pytest.mark.parametrize("T,H,F,E,K,skew", MOE_CASES, ids=["T%d-H%d-E%d-k%d%s" % (c[0], c[1], c[3], c[4],
                                                                                  "-skew" if c[5] else "")
                                                           for c in MOE_CASES])
def test_moe_prefill_vs_oracle(T, H, F, E, K, skew, dev):
    from lemoq import _hip

    print("case: moe_prefill T=%d H=%d F=%d E=%d k=%d skew=%s" % (T, H, F, E, K, skew), flush=True)
    x, router, gu_c, gu_s, dn_c, dn_s = _moe_case(T, H, F, E, K, T + H + E, dev, skew=skew)
    resid = randn(T, H, seed=T + 1).to(torch.float16)
    P, st = _hip.ptr, _hip.stream_of(dev)
    lib = _hip.load()
    f16 = dict(dtype=torch.float16, device=dev)
    i32 = dict(dtype=torch.int32, device=dev)
    xd, rd = x.to(dev), router.to(dev)
    gcd, gsd, dcd, dsd = gu_c.to(dev), gu_s.to(dev), dn_c.to(dev), dn_s.to(dev)
    rlog = torch.empty((T, E), **f16)
    top_w = torch.empty((T, K), dtype=torch.float32, device=dev)
    top_i = torch.empty((T, K), dtype=torch.int64, device=dev)
    pairs = T * K
    mt = int(lib.lemoq_moe_prefill_max_tiles(pairs, E))
    pair_tok, pair_src = torch.empty((pairs,), **i32), torch.empty((pairs,), **i32)
    pair_w, expert_off = torch.empty((pairs,), **f16), torch.empty((E + 1,), **i32)
    tiles = torch.full((mt, 4), -7, **i32)
    act = torch.empty((pairs, F), **f16)
    ybuf = torch.empty((pairs, H), **f16)
    out = resid.clone().to(dev)
    _hip.call("lemoq_gemm_f16", P(xd), T, H, H, P(rd), E, P(rlog), E, st)
    _hip.call("lemoq_route_topk", P(rlog), 1, T, E, E, K, 0, P(top_w), P(top_i), st)
    _hip.call("lemoq_moe_prefill_sort", P(top_i), P(top_w), T, K, E, P(pair_tok), P(pair_src), P(pair_w),
              P(expert_off), P(tiles), mt, st)
    _hip.call("lemoq_moe_prefill_gate_up", P(xd), H, P(pair_tok), P(tiles), mt, P(gcd), P(gsd), F, 128, P(act), st)
    _hip.call("lemoq_moe_prefill_down", P(act), F, P(pair_src), P(pair_w), P(tiles), mt, P(dcd), P(dsd), H, 128,
              P(ybuf), st)
    _hip.call("lemoq_moe_prefill_combine", P(ybuf), P(top_i), T, K, H, P(out), P(out), st)
    torch.cuda.synchronize()

    # the sort, exactly
    ti, tw = top_i.cpu(), top_w.cpu()
    flat = ti.reshape(-1)
    order = sorted(range(pairs), key=lambda p: (int(flat[p]), p))
    assert pair_src.cpu().tolist() == order
    assert pair_tok.cpu().tolist() == [p // K for p in order]
    assert torch.equal(pair_w.cpu(), tw.reshape(-1)[order].to(torch.float16))
    counts = torch.bincount(flat, minlength=E)
    assert expert_off.cpu().tolist() == [0] + torch.cumsum(counts, 0).tolist()
    tl = tiles.cpu()
    live = tl[tl[:, 0] >= 0]
    assert int((tl[:, 0] == -1).sum()) == mt - live.shape[0]
    covered = []
    for e_, b, en, _ in live.tolist():
        assert 0 < en - b <= 128 and int(flat[order[b]]) == e_ and int(flat[order[en - 1]]) == e_
        covered.extend(range(b, en))
    assert sorted(covered) == list(range(pairs))
    if skew:
        assert int(counts.max()) > 128

    moe = ops.moe_prefill_w8(x, gu_c, gu_s, dn_c, dn_s, 128, ti, tw.to(torch.float16))
    ref = (moe.float() + resid.float()).to(torch.float16)
    assert_close(out.cpu(), ref, what="moe_prefill T=%d" % T)


SORT_CASES = [(4096, 8, 64, "uniform"), (4096, 8, 64, "bench"), (1537, 3, 64, "uniform"), (2500, 8, 200, "skew"),
              (1, 1, 4, "uniform")]


@pytest.mark.parametrize("T,K,E,kind", SORT_CASES, ids=["T%d-k%d-E%d-%s" % c for c in SORT_CASES])
def test_moe_sort_exact(T, K, E, kind, dev):
    """The expert sort at the largest pair counts (several id batches per thread, the whole
    byte table in LDS) and ragged ones (pairs not a multiple of 4): the stable order, the
    fp16 routing weights, the expert offsets and the tile table, exactly.  "bench" routes
    every token to the same K experts (the bench's repeated prompt), "skew" half of them."""
    from lemoq import _hip

    print("case: moe_sort T=%d K=%d E=%d %s" % (T, K, E, kind), flush=True)
    g = torch.Generator().manual_seed(T * K + E)
    if kind == "bench":
        ti = torch.arange(K, dtype=torch.int64).repeat(T, 1) * 3 % E
    else:
        ti = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int64)
        if kind == "skew":
            ti[: T // 2] = torch.arange(K, dtype=torch.int64)
    tw = torch.rand((T, K), generator=g)
    pairs = T * K
    lib = _hip.load()
    mt = int(lib.lemoq_moe_prefill_max_tiles(pairs, E))
    i32 = dict(dtype=torch.int32, device=dev)
    pair_tok, pair_src = torch.full((pairs,), -5, **i32), torch.full((pairs,), -5, **i32)
    pair_w = torch.empty((pairs,), dtype=torch.float16, device=dev)
    expert_off = torch.full((E + 1,), -5, **i32)
    tiles = torch.full((mt, 4), -7, **i32)
    P, st = _hip.ptr, _hip.stream_of(dev)
    tid, twd = ti.to(dev), tw.to(dev)
    _hip.call("lemoq_moe_prefill_sort", P(tid), P(twd), T, K, E, P(pair_tok), P(pair_src), P(pair_w),
              P(expert_off), P(tiles), mt, st)
    torch.cuda.synchronize()
    flat = ti.reshape(-1)
    order = torch.from_numpy(np.argsort(flat.numpy(), kind="stable")).to(torch.int64)
    assert torch.equal(pair_src.cpu().to(torch.int64), order)
    assert torch.equal(pair_tok.cpu().to(torch.int64), order // K)
    assert torch.equal(pair_w.cpu(), tw.reshape(-1)[order].to(torch.float16))
    counts = torch.bincount(flat, minlength=E)
    assert expert_off.cpu().tolist() == [0] + torch.cumsum(counts, 0).tolist()
    tl = tiles.cpu()
    live = tl[tl[:, 0] >= 0]
    assert int((tl[:, 0] == -1).sum()) == mt - live.shape[0]
    assert live.shape[0] == int(((counts + 127) // 128).sum())
    sorted_ids = flat[order]
    covered = torch.zeros((pairs,), dtype=torch.int64)
    for e_, b, en, _ in live.tolist():
        assert 0 < en - b <= 128 and int(sorted_ids[b]) == e_ and int(sorted_ids[en - 1]) == e_
        covered[b:en] += 1
    assert bool((covered == 1).all())


@pytest.mark.parametrize("T,K", [(1, 8), (2, 8), (1, 2)])
def test_moe_prefill_small_table_blocks_equal_wide_blocks(T, K, dev):
    """A tile table of at most 16 entries runs 64-weight-row blocks (the last prompt row's MoE,
    called with max_tiles = its live tiles); the same sort output through the 256-row blocks
    (the full table) gives identical act and y bytes."""
    from lemoq import _hip

    H, F, E = 2048, 1024, 64
    print("case: moe small table T=%d K=%d" % (T, K), flush=True)
    x, router, gu_c, gu_s, dn_c, dn_s = _moe_case(T, H, F, E, K, 91 + T + K, dev)
    g = torch.Generator().manual_seed(T * 31 + K)
    ti = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int64)
    tw = torch.rand((T, K), generator=g)
    pairs = T * K
    mt = int(_hip.load().lemoq_moe_prefill_max_tiles(pairs, E))
    live = len(set(ti.reshape(-1).tolist()))  # one tile per expert here (under 128 pairs)
    assert live <= 16 < mt
    P, st = _hip.ptr, _hip.stream_of(dev)
    i32 = dict(dtype=torch.int32, device=dev)
    pair_tok, pair_src = torch.empty((pairs,), **i32), torch.empty((pairs,), **i32)
    pair_w = torch.empty((pairs,), dtype=torch.float16, device=dev)
    expert_off, tiles = torch.empty((E + 1,), **i32), torch.empty((mt, 4), **i32)
    xd, gcd, gsd, dcd, dsd = x.to(dev), gu_c.to(dev), gu_s.to(dev), dn_c.to(dev), dn_s.to(dev)
    _hip.call("lemoq_moe_prefill_sort", P(ti.to(dev)), P(tw.to(dev)), T, K, E, P(pair_tok), P(pair_src), P(pair_w),
              P(expert_off), P(tiles), mt, st)
    outs = []
    for m in (live, mt):
        act = torch.full((pairs, F), 3.0, dtype=torch.float16, device=dev)
        y = torch.full((pairs, H), 5.0, dtype=torch.float16, device=dev)
        _hip.call("lemoq_moe_prefill_gate_up", P(xd), H, P(pair_tok), P(tiles), m, P(gcd), P(gsd), F, 128, P(act), st)
        _hip.call("lemoq_moe_prefill_down", P(act), F, P(pair_src), P(pair_w), P(tiles), m, P(dcd), P(dsd), H, 128,
                  P(y), st)
        outs.append((act.cpu(), y.cpu()))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))
    assert torch.equal(outs[0][1].view(torch.int16), outs[1][1].view(torch.int16))
    assert not torch.isnan(outs[0][1].float()).any()


COMBINE_NORM_CASES = [(1, 2048, 8, True), (77, 2048, 8, True), (513, 4096, 2, True), (40, 8192, 8, False),
                      (9, 264, 4, True)]


@pytest.mark.parametrize("T,H,K,with_resid", COMBINE_NORM_CASES,
                         ids=["T%d-H%d-k%d%s" % (c[0], c[1], c[2], "-resid" if c[3] else "")
                              for c in COMBINE_NORM_CASES])
def test_moe_combine_norm_equals_combine_then_rmsnorm(T, H, K, with_resid, dev):
    """The combine that also writes the next layer's input norm gives the plain combine's rows and
    lemoq_rmsnorm's norm of them, bit for bit; the norm also against the oracle's RMSNorm."""
    from lemoq import _hip

    print("case: combine_norm T=%d H=%d k=%d resid=%s" % (T, H, K, with_resid), flush=True)
    P, st = _hip.ptr, _hip.stream_of(dev)
    gen = torch.Generator().manual_seed(T * H + K)
    y = (torch.randn((T * K, H), generator=gen) * 0.5).to(torch.float16).to(dev)
    top_i = torch.stack([torch.randperm(64, generator=gen)[:K] for _ in range(T)]).to(torch.int64).to(dev)
    resid = (torch.randn((T, H), generator=gen) * 2.0).to(torch.float16).to(dev)
    w = (1.0 + 0.1 * torch.randn((H,), generator=gen)).to(torch.float16).to(dev)
    eps = 1e-5
    out_a = resid.clone()
    out_b = resid.clone()
    xn_a = torch.full((T, H), 7.0, dtype=torch.float16, device=dev)
    xn_b = torch.full((T, H), 9.0, dtype=torch.float16, device=dev)
    rp = P(out_a) if with_resid else None
    _hip.call("lemoq_moe_prefill_combine", P(y), P(top_i), T, K, H, rp, P(out_a), st)
    _hip.call("lemoq_rmsnorm", P(out_a), T, H, P(w), eps, P(xn_a), st)
    rp = P(out_b) if with_resid else None
    _hip.call("lemoq_moe_prefill_combine_norm", P(y), P(top_i), T, K, H, rp, P(out_b), P(w), eps, P(xn_b), st)
    torch.cuda.synchronize()
    assert torch.equal(out_a.cpu(), out_b.cpu())
    assert torch.equal(xn_a.cpu(), xn_b.cpu())
    assert_close(xn_b.cpu(), ops.rms_norm(out_b.cpu(), w.cpu(), eps), what="combine_norm T=%d H=%d" % (T, H))


def _prefill_vs_oracle(shape, prompt, seed, steps, dev):
    from lemoq.model.olmoe import DecodeSession, OlmoeW8Weights

    w = OlmoeW8Weights.random(shape, seed=seed, device=dev)
    sess = DecodeSession(w, prompt, max_new_tokens=steps, num_splits=None)
    rows = []
    seed_tok = sess.prefill(kv_f16=rows)
    logits = sess.logits_cpu()
    kv = sess.kv_cpu()
    hw = w.to_host()
    ref_rows = []
    ref, ref_kv = oracle_prefill(hw, prompt, sess.max_seq, kv_f16=ref_rows)
    ref64, got64 = ref.double(), logits.double()
    p, q = torch.log_softmax(ref64, -1), torch.log_softmax(got64, -1)
    kl = float((p.exp() * (p - q)).sum())
    diff = float((ref64 - got64).abs().max())
    print("prefill T=%d: KL %.2e, max|diff| %.3e (max|logit| %.2f)" % (len(prompt), kl, diff,
                                                                      float(ref64.abs().max())))
    assert kl < 1e-2 and diff <= 2e-2 * float(ref64.abs().max())
    if seed_tok != int(torch.argmax(ref64)):
        top = torch.topk(ref64, 2).values
        assert float(top[0] - top[1]) <= 2 * diff
    T = len(prompt)
    assert len(rows) == len(ref_rows) == shape.layers
    for li in range(shape.layers):
        kv_rows_vs_oracle("prefill T=%d layer %d" % (T, li), kv[li], rows[li], ref_kv[li], ref_rows[li], T,
                          rows_close=li == 0)
    assert sess.position == T and sess.generated() == [seed_tok]
    # decode from the prefilled cache, checked step by step against the CPU decoder on the same cache
    gl = []
    for _ in range(steps):
        sess.replay(1)
        gl.append(sess.logits_cpu())
    toks = [int(t) for t in sess.history[T: T + steps + 1].tolist()]
    oracle = OracleDecoder(hw, sess.max_seq, kv=kv)
    for i in range(steps):
        r = oracle.step(toks[i], T + i).double()
        gq = gl[i].double()
        pr, qr = torch.log_softmax(r, -1), torch.log_softmax(gq, -1)
        assert float((pr.exp() * (pr - qr)).sum()) < 1e-2, i
        assert float((r - gq).abs().max()) <= 2e-2 * float(r.abs().max()), i


def test_prefill_session_tiny(dev):
    from lemoq.model.olmoe import OlmoeShape

    print("case: prefill session tiny", flush=True)
    shape = OlmoeShape(hidden=512, heads=4, head_dim=128, layers=2, num_experts=8, top_k=2, ffn=256, vocab=1024)
    prompt = [int(t) for t in torch.randint(0, 1024, (45,), generator=torch.Generator().manual_seed(8))]
    _prefill_vs_oracle(shape, prompt, 3, 6, dev)


def test_prefill_session_clip_qkv(dev):
    """A model with HF OLMoE's clip_qkv set: the batched prefill (rows kernel)
    and the decode steps after it (fused attention launch) against the oracles
    with the same clamp."""
    from lemoq.model.olmoe import OlmoeShape

    print("case: prefill session tiny, clip_qkv 0.8", flush=True)
    shape = OlmoeShape(hidden=512, heads=4, head_dim=128, layers=2, num_experts=8, top_k=2, ffn=256, vocab=1024,
                       clip_qkv=0.8)
    prompt = [int(t) for t in torch.randint(0, 1024, (45,), generator=torch.Generator().manual_seed(18))]
    _prefill_vs_oracle(shape, prompt, 3, 6, dev)


def test_prefill_session_olmoe_shape(dev):
    from lemoq.model.olmoe import OLMOE_1B_7B

    print("case: prefill session OLMoE-1B-7B T=64", flush=True)
    prompt = [int(t) for t in torch.randint(0, OLMOE_1B_7B.vocab, (64,), generator=torch.Generator().manual_seed(9))]
    _prefill_vs_oracle(OLMOE_1B_7B, prompt, 4, 4, dev)


def test_prefill_modes_agree_on_the_canonical_prompt(dev):
    """Batched and stepped prefill of ctx ones: the same seed token unless near-tied, close logits."""
    from lemoq.model.olmoe import DecodeSession, OlmoeShape, OlmoeW8Weights

    print("case: prefill modes", flush=True)
    shape = OlmoeShape(hidden=512, heads=4, head_dim=128, layers=2, num_experts=8, top_k=2, ffn=256, vocab=1024)
    w = OlmoeW8Weights.random(shape, seed=12, device=dev)
    sess = DecodeSession(w, [1] * 33, max_new_tokens=2, num_splits=None)
    a = sess.prefill()
    la = sess.logits_cpu().double()
    b = sess.prefill(mode="stepped")
    lb = sess.logits_cpu().double()
    diff = float((la - lb).abs().max())
    assert diff <= 3e-2 * float(lb.abs().max())
    if a != b:
        top = torch.topk(lb, 2).values
        assert float(top[0] - top[1]) <= 2 * diff


@pytest.mark.parametrize("T", [2, 300, 1024])
def test_prefill_last_layer_on_the_last_row_only(T, dev):
    """The last layer run on the last position only (after its KV rows are written for every
    position) against the same layer run on every position: identical KV-INT8 caches (the rows
    come from the same launches), the last logits within the fp16 tolerance of each other and
    the same seed token unless the two top logits are within that difference."""
    from lemoq.kernels.rope import rotary_cos_sin
    from lemoq.model.olmoe import OlmoeShape, OlmoeW8Weights
    from lemoq.model.prefill import prefill_prompt

    print("case: prefill last row only T=%d" % T, flush=True)
    shape = OlmoeShape(hidden=512, heads=4, head_dim=128, layers=3, num_experts=16, top_k=4, ffn=256, vocab=4096)
    w = OlmoeW8Weights.random(shape, seed=T, device=dev)
    S = T + 8
    cos, sin = (t.to(dev).contiguous() for t in rotary_cos_sin(torch.arange(S), shape.head_dim, shape.rope_theta))
    g = torch.Generator().manual_seed(T)
    tokens = torch.randint(0, shape.vocab, (T,), generator=g).to(torch.int64).to(dev)
    outs = []
    for last_only in (True, False):
        kv = [{"kc": torch.zeros((shape.heads, S, shape.head_dim), dtype=torch.int8, device=dev),
               "ks": torch.zeros((shape.heads, S), dtype=torch.float16, device=dev),
               "vc": torch.zeros((shape.heads, S, shape.head_dim), dtype=torch.int8, device=dev),
               "vs": torch.zeros((shape.heads, S), dtype=torch.float16, device=dev)} for _ in range(shape.layers)]
        logits = torch.empty((shape.vocab,), dtype=torch.float16, device=dev)
        step = {"token": torch.zeros((1,), dtype=torch.int64, device=dev),
                "pos": torch.full((1,), T - 1, dtype=torch.int64, device=dev),
                "filled": torch.zeros((1,), dtype=torch.int32, device=dev),
                "history": torch.zeros((S,), dtype=torch.int64, device=dev)}
        prefill_prompt(w, tokens, kv, cos, sin, S, logits, step=step, last_row_only=last_only)
        torch.cuda.synchronize()
        outs.append((kv, logits.cpu(), int(step["token"].item())))
    (kv_a, lg_a, tok_a), (kv_b, lg_b, tok_b) = outs
    for la, lb in zip(kv_a, kv_b):
        for name in ("kc", "ks", "vc", "vs"):
            assert torch.equal(la[name].cpu(), lb[name].cpu()), name
    assert_close(lg_a, lg_b, what="last logits T=%d" % T)
    if tok_a != tok_b:
        top = torch.topk(lg_b.float(), 2).values
        assert float(top[0] - top[1]) <= float((lg_a.float() - lg_b.float()).abs().max())
