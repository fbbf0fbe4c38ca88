"""GPU parity of the floating-point operators against the CPU oracle.

Cases mirror the reference's K1 gates: tests/test_kernel_parity.py:134-282
(dequant GEMV m in {1,4}, k in {2048,256,500,512,1024}; grouped MoE vs fp64),
tests/test_attn_decode.py:421-494 and tests/test_fusion_adversarial.py:72-85
(split-KV vs fp64, filled in {0,1,17}, NaN tail, length change),
tests/test_kv_int8_read_gpu.py:90-146 (int8 attention vs dequant fp64),
tests/test_rmsnorm_parity.py:31-58, tests/test_fused_rope.py:114-143,
tests/test_routing_fusion.py:72-119, tests/test_packed_qkv.py:152-174.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import ATOL, RTOL, assert_close, assert_gate, max_abs, randn
from oracle import ops
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def _q8(w: torch.Tensor, group: int):
    q = oq.rtn_quantize_w8(w.numpy(), group)
    return torch.from_numpy(q["codes_padded"]), torch.from_numpy(q["scale_f16"])


# ---------------------------------------------------------------------------
# dense w8 GEMV
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("k", [2048, 256, 500, 512, 1024])
def test_dequant_gemm_fused_vs_fp64(m, k, dev):
    from lemoq.kernels.dequant_gemm import dequant_gemm_fused

    n = 384
    group = 128
    w = randn(n, k, seed=k + m, std=0.02)
    codes, scale = _q8(w, group)
    x = (randn(m, k, seed=7 * k + m) * 0.5).to(torch.float16)
    w64 = ops.dequant_w8(codes, scale, group)[:, :k].double()
    ref64 = x.double() @ w64.t()
    # fp32 output: the reference's K1 gate against the separate (dequantise-then-GEMM) arm
    got32 = dequant_gemm_fused(x.to(dev), codes.to(dev), scale.to(dev), None, group_size=group, bits=8)
    assert got32.dtype == torch.float32
    baseline = ops.dequant_gemm_separate(x, codes, scale, group)
    assert_gate(got32.cpu(), ref64, baseline, what="gemv fp32 m=%d k=%d" % (m, k))
    # fp16 output (the decode path): rtol 2e-2 / atol 2e-3 against fp64
    got = dequant_gemm_fused(x.to(dev), codes.to(dev), scale.to(dev), None, group_size=group,
                             bits=8, out_dtype=torch.float16)
    assert_close(got.cpu(), ref64, what="gemv fp16 m=%d k=%d" % (m, k))
    assert torch.equal(got.cpu(), got32.cpu().to(torch.float16))


@pytest.mark.parametrize("n", [6144, 2048, 50304])
def test_dequant_gemm_olmoe_shapes(n, dev):
    from lemoq.kernels.dequant_gemm import dequant_gemm_fused

    k = 2048
    w = randn(n, k, seed=n, std=0.02)
    codes, scale = _q8(w, 128)
    x = randn(1, k, seed=n + 1).to(torch.float16)
    got = dequant_gemm_fused(x.to(dev), codes.to(dev), scale.to(dev), None, group_size=128,
                             bits=8, out_dtype=torch.float16).cpu()
    ref = ops.dequant_gemm_fused_tiles(x, codes, scale, 128)
    assert_close(got, ref, what="gemv N=%d" % n)


def test_packed_qkv_bitwise_equals_three_calls(dev):
    from lemoq.kernels.packed_qkv import pack_qkv
    from lemoq.quant.linear import QuantLinear

    projs = [QuantLinear(randn(2048, 2048, seed=s, std=0.02).to(dev)) for s in (1, 2, 3)]
    packed = pack_qkv(*projs)
    x = randn(1, 1, 2048, seed=9).to(torch.float16).to(dev)
    q, k, v = packed.project(x)
    for got, proj in zip((q, k, v), projs):
        assert torch.equal(got, proj(x))


def test_gemv_fused_norm_and_residual(dev):
    from lemoq import _hip

    H, N = 2048, 2048
    w = randn(N, H, seed=21, std=0.02)
    codes, scale = _q8(w, 128)
    x = randn(H, seed=22).to(torch.float16)
    gamma = (torch.rand(H, generator=torch.Generator().manual_seed(23)) + 0.5).to(torch.float16)
    resid = randn(N, seed=24).to(torch.float16)
    y = resid.clone().to(dev)
    # keep every device tensor referenced until the kernel has run
    xd, gd, cd, sd = x.to(dev), gamma.to(dev), codes.to(dev), scale.to(dev)
    _hip.call("lemoq_gemv_w8_fused", _hip.ptr(xd), None, 0, _hip.ptr(gd), 1e-5, None,
              _hip.ptr(cd), _hip.ptr(sd), N, H, 128, _hip.ptr(y), _hip.ptr(y), _hip.stream_of(dev))
    torch.cuda.synchronize()
    xn = ops.rms_norm(x, gamma, 1e-5)
    ref = (ops.dequant_gemm_separate(xn.reshape(1, -1), codes, scale, 128).reshape(-1)
           .to(torch.float16) + resid)
    assert_close(y.cpu(), ref, what="norm+gemv+residual")


# ---------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("e,k", [(64, 8), (12, 3), (8, 8), (100, 5)])
def test_routing_softmax_topk_vs_oracle(norm, e, k, dev):
    from lemoq.kernels.routing import routing_softmax_topk

    logits = randn(7, e, seed=e * 10 + k)
    ref_w, ref_i = oq.route_order(logits.numpy(), k, norm)
    got_w, got_i = routing_softmax_topk(logits.to(dev), top_k=k, norm_topk_prob=norm)
    assert np.array_equal(got_i.cpu().numpy(), ref_i)
    assert np.allclose(got_w.cpu().numpy(), ref_w, atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("case", ["all_equal", "kth_boundary", "fp16_rounding"])
def test_routing_ties_lowest_index(case, dev):
    from lemoq.kernels.routing import routing_softmax_topk

    logits = torch.zeros(1, 64)
    if case == "kth_boundary":
        logits[:, :7] = torch.arange(8, 1, -1).float()
    elif case == "fp16_rounding":
        logits = (torch.ones_like(logits) + torch.arange(64) * 1e-6).half().float()
    ref_w, ref_i = oq.route_order(logits.numpy(), 8, False)
    got_w, got_i = routing_softmax_topk(logits.to(dev), top_k=8)
    assert np.array_equal(got_i.cpu().numpy(), ref_i), (case, got_i, ref_i)
    assert np.allclose(got_w.cpu().numpy(), ref_w, atol=1e-6)


@pytest.mark.parametrize("norm", [False, True])
def test_fused_router_vs_oracle(norm, dev):
    from lemoq.kernels.moe_static import _route

    for seed in range(8):
        x = randn(1, 2048, seed=100 + seed).to(torch.float16)
        rw = randn(64, 2048, seed=200 + seed, std=0.02).to(torch.float16)
        lg, tw, ti = _route(x.to(dev), rw.to(dev), top_k=8, norm_topk_prob=norm)
        rlg, rtw, rti = ops.route(x, rw, 8, norm)
        # logits: one fp16 rounding of an fp32 dot; summation order may move a value by 1 ulp
        assert max_abs(lg.cpu(), rlg) <= 2e-3
        assert np.array_equal(ti.cpu().numpy(), rti.numpy()), seed
        assert torch.allclose(tw.cpu().float(), rtw.float(), atol=1e-3, rtol=0)
        assert tw.dtype == torch.float16 and ti.dtype == torch.int64


@pytest.mark.parametrize("T", [2, 7, 64])
@pytest.mark.parametrize("norm", [False, True])
def test_route_several_tokens_vs_oracle(T, norm, dev):
    """``_route`` on several fp16 tokens (the prefill shape) runs the router linear
    as lemoq_gemm_f16 and the HIP top-k: logits against the oracle's F.linear
    (one fp16 rounding of an fp32 dot; the order may move a value by one ulp),
    the ids bit-exact against the oracle's top-k of the GPU's own logits (ties
    -> lowest index), so a near-tied pair cannot excuse a wrong selection, and
    the weights within 1e-3 (fp32 softmax, then fp16)."""
    from lemoq.kernels.moe_static import _route

    print("case: _route T=%d norm=%s" % (T, norm), flush=True)
    x = randn(T, 2048, seed=300 + T).to(torch.float16)
    rw = randn(64, 2048, seed=400 + T, std=0.02).to(torch.float16)
    lg, tw, ti = _route(x.to(dev), rw.to(dev), top_k=8, norm_topk_prob=norm)
    rlg, _, _ = ops.route(x, rw, 8, norm)
    assert lg.shape == (T, 64) and tw.shape == (T, 8) and ti.shape == (T, 8)
    assert max_abs(lg.cpu(), rlg) <= 2e-3
    gw, gi = ops.route_logits(lg.cpu(), 8, norm)
    assert np.array_equal(ti.cpu().numpy(), gi.numpy())
    assert torch.allclose(tw.cpu().float(), gw.float(), atol=1e-3, rtol=0)
    assert tw.dtype == torch.float16 and ti.dtype == torch.int64


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("E", [64, 8, 100])
def test_router_logits_then_routed_gate_up_vs_oracle(norm, E, dev):
    """The decode step's routing path: lemoq_router_logits (one wave per expert)
    then the routing inside lemoq_moe_gate_up_w8_routed.  ids must equal the
    oracle's _route bit for bit; act must equal the plain gate/up on those ids."""
    from lemoq import _hip

    H, F, K, g = 2048, 256, min(8, E), 128
    gc, gs, _, _ = _experts(E, F, H, g, seed=300 + E)
    for seed in range(6):
        h = randn(H, seed=400 + seed).to(torch.float16)
        ln = (torch.rand(H, generator=torch.Generator().manual_seed(seed)) + 0.5).to(torch.float16)
        rw = randn(E, H, seed=500 + seed, std=0.02).to(torch.float16)
        hd, lnd, rwd = h.to(dev), ln.to(dev), rw.to(dev)
        xn = torch.empty(H, dtype=torch.float16, device=dev)
        lg = torch.empty(E, dtype=torch.float16, device=dev)
        st = _hip.stream_of(dev)
        _hip.call("lemoq_router_logits", _hip.ptr(hd), _hip.ptr(lnd), 1e-5, H, _hip.ptr(rwd), E,
                  _hip.ptr(xn), _hip.ptr(lg), st)
        xn_ref = ops.rms_norm(h, ln, 1e-5)
        assert max_abs(xn.cpu(), xn_ref) <= 2e-3
        rlg, rtw, rti = ops.route(xn_ref.reshape(1, H), rw, K, norm)
        assert max_abs(lg.cpu(), rlg.reshape(-1)) <= 2e-3
        act = torch.empty(K, F, dtype=torch.float16, device=dev)
        ti = torch.empty(K, dtype=torch.int64, device=dev)
        tw = torch.empty(K, dtype=torch.float16, device=dev)
        gcd, gsd = gc.to(dev), gs.to(dev)
        _hip.call("lemoq_moe_gate_up_w8_routed", _hip.ptr(xn), _hip.ptr(gcd), _hip.ptr(gsd), _hip.ptr(lg), K,
                  1 if norm else 0, E, F, H, g, _hip.ptr(act), _hip.ptr(ti), _hip.ptr(tw), st)
        # routing of the GPU logits by the oracle's rule: bit-exact ids
        ref_w, ref_i = oq.route_order(lg.cpu().float().numpy()[None], K, norm)
        assert np.array_equal(ti.cpu().numpy(), ref_i[0]), seed
        assert torch.allclose(tw.cpu().float(), torch.from_numpy(ref_w[0]).half().float(), atol=1e-3, rtol=0)
        act2 = torch.empty_like(act)
        _hip.call("lemoq_moe_gate_up_w8", _hip.ptr(xn), _hip.ptr(gcd), _hip.ptr(gsd), _hip.ptr(ti), K, E, F, H, g,
                  _hip.ptr(act2), st)
        assert torch.equal(act, act2)


@pytest.mark.parametrize("case", ["ties_inside", "ties_at_boundary", "all_equal", "descending"])
@pytest.mark.parametrize("norm", [False, True])
def test_routed_gate_up_with_tied_logits(case, norm, dev):
    """Every block of lemoq_moe_gate_up_w8_routed selects its own slot's expert
    (argmax rounds up to its rank): with tied logits the ids must follow the
    oracle's order (larger first, ties -> lower index) for every slot, and act
    must equal the plain gate/up on the oracle's ids."""
    from lemoq import _hip

    E, K, H, F, g = 64, 8, 2048, 256, 128
    gc, gs, _, _ = _experts(E, F, H, g, seed=910)
    z = torch.linspace(-2.0, 1.0, E)[torch.randperm(E, generator=torch.Generator().manual_seed(3))]
    if case == "ties_inside":
        z[[5, 9, 40]] = 3.0   # three-way tie at the top
        z[[2, 33]] = 2.5
    elif case == "ties_at_boundary":
        z[:6] = torch.tensor([4.0, 3.9, 3.8, 3.7, 3.6, 3.5])
        z[[10, 20, 30, 50]] = 3.0  # ranks 6..9 tie: only 10 and 20 are selected
    elif case == "all_equal":
        z[:] = 0.5
    else:
        z = torch.linspace(2.0, -2.0, E)
    lg = z.to(torch.float16)
    x = randn(H, seed=911).to(torch.float16)
    st = _hip.stream_of(dev)
    gcd, gsd, xd, lgd = gc.to(dev), gs.to(dev), x.to(dev), lg.to(dev)
    act = torch.empty(K, F, dtype=torch.float16, device=dev)
    ti = torch.empty(K, dtype=torch.int64, device=dev)
    tw = torch.empty(K, dtype=torch.float16, device=dev)
    _hip.call("lemoq_moe_gate_up_w8_routed", _hip.ptr(xd), _hip.ptr(gcd), _hip.ptr(gsd), _hip.ptr(lgd), K,
              1 if norm else 0, E, F, H, g, _hip.ptr(act), _hip.ptr(ti), _hip.ptr(tw), st)
    ref_w, ref_i = oq.route_order(lg.float().numpy()[None], K, norm)
    assert np.array_equal(ti.cpu().numpy(), ref_i[0]), (case, ti.cpu().tolist(), ref_i[0].tolist())
    assert torch.allclose(tw.cpu().float(), torch.from_numpy(ref_w[0]).half().float(), atol=1e-3, rtol=0)
    ids = torch.from_numpy(ref_i[0].astype(np.int64)).to(dev)
    act2 = torch.empty_like(act)
    _hip.call("lemoq_moe_gate_up_w8", _hip.ptr(xd), _hip.ptr(gcd), _hip.ptr(gsd), _hip.ptr(ids), K, E, F, H, g,
              _hip.ptr(act2), st)
    assert torch.equal(act, act2), case


# ---------------------------------------------------------------------------
# grouped MoE
# ---------------------------------------------------------------------------
def _experts(E, F, H, group, seed):
    gu = randn(E * 2 * F, H, seed=seed, std=0.02)
    dn = randn(E * H, F, seed=seed + 1, std=0.02)
    gc, gs = _q8(gu, group)
    dc, ds = _q8(dn, group)
    return (gc.reshape(E, 2 * F, H), gs.reshape(E, 2 * F, H // group),
            dc.reshape(E, H, F), ds.reshape(E, H, F // group))


@pytest.mark.parametrize("E,F,H,K", [(64, 1024, 2048, 8), (8, 256, 512, 2), (16, 128, 1024, 4)])
def test_grouped_moe_vs_fp64(E, F, H, K, dev):
    from lemoq.kernels.moe_grouped_quant import QuantFusedExperts, grouped_moe_forward_quant

    gc, gs, dc, ds = _experts(E, F, H, 128, seed=E + F)
    q = QuantFusedExperts(gc.to(dev), gs.to(dev), dc.to(dev), ds.to(dev), bits=8, group_size=128)
    x = randn(H, seed=3).to(torch.float16)
    ids = torch.randperm(E, generator=torch.Generator().manual_seed(4))[:K]
    w = torch.softmax(randn(K, seed=5), 0).to(torch.float16)
    got = grouped_moe_forward_quant(x.to(dev), q, ids.to(dev), w.to(dev)).cpu()
    ref, act_ref = ops.grouped_moe_w8(x, gc, gs, dc, ds, 128, ids, w)
    # fp64 closed form on the dequantised weights with the fp16 act rounding point
    gu64 = torch.stack([ops.dequant_w8(gc[e], gs[e], 128) for e in ids.tolist()]).double()
    g = gu64[:, :F] @ x.double()
    u = gu64[:, F:] @ x.double()
    act64 = (g * torch.sigmoid(g) * u).to(torch.float16).double()
    dn64 = torch.stack([ops.dequant_w8(dc[e], ds[e], 128) for e in ids.tolist()]).double()
    out64 = ((dn64 @ act64.unsqueeze(-1)).squeeze(-1) * w.double().unsqueeze(1)).sum(0)
    assert_close(got, out64, what="moe vs fp64")
    assert_close(got, ref, what="moe vs oracle")


def _moe_fp64(x, gc, gs, dc, ds, ids, w, F):
    gu64 = torch.stack([ops.dequant_w8(gc[e], gs[e], 128) for e in ids.tolist()]).double()
    g, u = gu64[:, :F] @ x.double(), gu64[:, F:] @ x.double()
    act64 = (g * torch.sigmoid(g) * u).to(torch.float16).double()
    dn64 = torch.stack([ops.dequant_w8(dc[e], ds[e], 128) for e in ids.tolist()]).double()
    return ((dn64 @ act64.unsqueeze(-1)).squeeze(-1) * w.double().unsqueeze(1)).sum(0)


@pytest.mark.parametrize("E,F,H,K", [(64, 1024, 2048, 8), (8, 256, 512, 4)])
def test_grouped_moe_degenerate_routing_all_slots_same_expert(E, F, H, K, dev):
    """Every slot routed to one expert (the reference's
    tests/test_moe_grouped.py:139-153): the slots' gate/up and down rows are
    the same rows, summed over the slots in fixed order with their own weights."""
    from lemoq.kernels.moe_grouped_quant import QuantFusedExperts, grouped_moe_forward_quant

    gc, gs, dc, ds = _experts(E, F, H, 128, seed=E + 3 * F)
    q = QuantFusedExperts(gc.to(dev), gs.to(dev), dc.to(dev), ds.to(dev), bits=8, group_size=128)
    x = randn(H, seed=41).to(torch.float16)
    for e in (0, E - 1, E // 3):
        ids = torch.full((K,), e, dtype=torch.int64)
        w = torch.softmax(randn(K, seed=42 + e), 0).to(torch.float16)
        got = grouped_moe_forward_quant(x.to(dev), q, ids.to(dev), w.to(dev)).cpu()
        ref, _ = ops.grouped_moe_w8(x, gc, gs, dc, ds, 128, ids, w)
        assert_close(got, _moe_fp64(x, gc, gs, dc, ds, ids, w, F), what="expert %d x%d vs fp64" % (e, K))
        assert_close(got, ref, what="expert %d x%d vs oracle" % (e, K))
        # one slot with the summed weight gives the same answer up to the fp16
        # rounding of that sum and of the output
        one = grouped_moe_forward_quant(x.to(dev), q, ids[:1].to(dev),
                                        w.float().sum().reshape(1).to(torch.float16).to(dev)).cpu()
        assert_close(got, one, rtol=5e-3, atol=1e-3, what="expert %d: x%d against one slot" % (e, K))


def test_grouped_moe_across_random_routings(dev):
    """Twelve seeded routings at one shape, each against the fp64 closed form
    and the oracle (the reference's tests/test_moe_grouped.py:123-137)."""
    from lemoq.kernels.moe_grouped_quant import QuantFusedExperts, grouped_moe_forward_quant

    E, F, H, K = 32, 256, 1024, 8
    gc, gs, dc, ds = _experts(E, F, H, 128, seed=51)
    q = QuantFusedExperts(gc.to(dev), gs.to(dev), dc.to(dev), ds.to(dev), bits=8, group_size=128)
    for s in range(12):
        g = torch.Generator().manual_seed(600 + s)
        x = (torch.randn(H, generator=g) * (0.5 + s / 4)).to(torch.float16)
        ids = torch.randperm(E, generator=g)[:K] if s % 3 else torch.randint(0, E, (K,), generator=g)
        w = torch.softmax(torch.randn(K, generator=g), 0).to(torch.float16)
        got = grouped_moe_forward_quant(x.to(dev), q, ids.to(dev), w.to(dev)).cpu()
        ref, _ = ops.grouped_moe_w8(x, gc, gs, dc, ds, 128, ids, w)
        assert_close(got, _moe_fp64(x, gc, gs, dc, ds, ids, w, F), what="routing %d vs fp64" % s)
        assert_close(got, ref, what="routing %d vs oracle" % s)


def test_grouped_moe_linear_in_weights_and_residual(dev):
    from lemoq.kernels.moe_grouped_quant import QuantFusedExperts, grouped_moe_forward_quant

    E, F, H, K = 8, 256, 512, 2
    gc, gs, dc, ds = _experts(E, F, H, 128, seed=77)
    q = QuantFusedExperts(gc.to(dev), gs.to(dev), dc.to(dev), ds.to(dev), bits=8, group_size=128)
    x = randn(H, seed=8).to(torch.float16).to(dev)
    ids = torch.tensor([5, 2], device=dev)
    w1 = torch.tensor([0.25, 0.5], dtype=torch.float16, device=dev)
    y1 = grouped_moe_forward_quant(x, q, ids, w1).float()
    y2 = grouped_moe_forward_quant(x, q, ids, w1 * 2).float()
    assert_close(y2.cpu(), 2 * y1.cpu(), rtol=2e-3, atol=1e-4, what="linearity")
    zero = grouped_moe_forward_quant(x, q, ids, torch.zeros_like(w1))
    assert (zero == 0).all()
    resid = randn(H, seed=9).to(torch.float16).to(dev)
    yr = grouped_moe_forward_quant(x, q, ids, w1, residual=resid)
    assert torch.equal(yr, (grouped_moe_forward_quant(x, q, ids, w1) + resid))


def test_static_moe_forward_block(dev):
    from lemoq.kernels.moe_grouped_quant import QuantFusedExperts, static_moe_forward_grouped_quant

    E, F, H = 64, 1024, 2048
    gc, gs, dc, ds = _experts(E, F, H, 128, seed=31)
    q = QuantFusedExperts(gc.to(dev), gs.to(dev), dc.to(dev), ds.to(dev), bits=8, group_size=128)
    x = randn(1, 1, H, seed=32).to(torch.float16)
    rw = randn(E, H, seed=33, std=0.02).to(torch.float16)
    for norm in (False, True):
        out, logits = static_moe_forward_grouped_quant(x.to(dev), rw.to(dev), q, top_k=8,
                                                      norm_topk_prob=norm, act_fn=torch.nn.functional.silu)
        rl, rw8, ri = ops.route(x.reshape(1, H), rw, 8, norm)
        ref, _ = ops.grouped_moe_w8(x.reshape(-1), gc, gs, dc, ds, 128, ri, rw8)
        assert out.shape == (1, 1, H)
        assert_close(out.cpu().reshape(-1), ref, what="static block norm=%s" % norm)


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
def _qkv(H, S, D, seed, qs=1.0):
    q = randn(1, H, 1, D, seed=seed, std=qs).to(torch.float16)
    k = randn(1, H, S, D, seed=seed + 1).to(torch.float16)
    v = randn(1, H, S, D, seed=seed + 2).to(torch.float16)
    return q, k, v


@pytest.mark.parametrize("ctx", [1024, 4096])
def test_attn_fp16_vs_fp64(ctx, dev):
    from lemoq.kernels.attn_decode import attn_decode_forward

    q, k, v = _qkv(16, ctx, 128, seed=ctx)
    n = torch.tensor([ctx], dtype=torch.int32, device=dev)
    got = attn_decode_forward(q.to(dev), k.to(dev), v.to(dev), n).cpu().reshape(16, 128)
    ref64 = ops.dense_attention(q.reshape(16, 128), k[0], v[0], ctx)
    base = ops.split_kv_oracle(q.reshape(16, 128), k[0], v[0], ctx, num_splits=11).to(torch.float16)
    assert_gate(got, ref64, base, what="attn fp16 ctx=%d" % ctx)


@pytest.mark.parametrize("splits", [1, 2, 3, 8, 17, 64, 65, 100])
def test_attn_split_count_invariance(splits, dev):
    from lemoq.kernels.attn_decode import attn_decode_forward

    q, k, v = _qkv(4, 700, 128, seed=50)
    n = torch.tensor([613], dtype=torch.int32, device=dev)
    got = attn_decode_forward(q.to(dev), k.to(dev), v.to(dev), n, config={"num_splits": splits})
    ref = ops.dense_attention(q.reshape(4, 128), k[0], v[0], 613)
    assert_close(got.cpu().reshape(4, 128), ref, rtol=1e-3, atol=1e-3, what="splits=%d" % splits)


@pytest.mark.parametrize("filled", [0, 1, 17])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_attn_length_boundaries(filled, D, dev):
    from lemoq.kernels.attn_decode import attn_decode_forward

    q, k, v = _qkv(2, 17, D, seed=60 + D, qs=0.1)
    n = torch.tensor([filled], dtype=torch.int32, device=dev)
    got = attn_decode_forward(q.to(dev), k.to(dev), v.to(dev), n, config={"num_splits": 4})
    ref = ops.dense_attention(q.reshape(2, D), k[0], v[0], filled).to(torch.float16)
    assert torch.isfinite(got).all()
    assert_close(got.cpu().reshape(2, D), ref, rtol=1e-3, atol=1e-3, what="filled=%d" % filled)
    if filled == 0:
        assert (got == 0).all()


def test_attn_nan_tail_never_read(dev):
    from lemoq.kernels.attn_decode import attn_decode_forward, attn_decode_forward_int8
    from lemoq.kernels.kv_int8 import kv_int8_bulk_quantize

    q, k, v = _qkv(16, 256, 128, seed=70)
    k[:, :, 100:] = float("nan")
    v[:, :, 100:] = float("nan")
    n = torch.tensor([100], dtype=torch.int32, device=dev)
    got = attn_decode_forward(q.to(dev), k.to(dev), v.to(dev), n)
    assert torch.isfinite(got).all()
    ref = ops.dense_attention(q.reshape(16, 128), k[0], v[0], 100)
    assert_close(got.cpu().reshape(16, 128), ref, what="nan tail fp16")
    bufs = kv_int8_bulk_quantize(k.to(dev), v.to(dev), filled=100)
    bufs["ks"][0, :, 100:] = float("nan")
    bufs["vs"][0, :, 100:] = float("nan")
    got8 = attn_decode_forward_int8(q.to(dev), bufs["kc"], bufs["ks"], bufs["vc"], bufs["vs"], n)
    assert torch.isfinite(got8).all()


def test_attn_length_change_is_read_on_device(dev):
    from lemoq.kernels.attn_decode import attn_decode_forward, judge_length_change

    q, k, v = _qkv(16, 2048, 128, seed=80)
    k[:, :, 1500:] *= 3.0  # make the late keys matter
    v[:, :, 1500:] += 4.0
    n = torch.tensor([1000], dtype=torch.int32, device=dev)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = attn_decode_forward(qd, kd, vd, n)  # warm
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = attn_decode_forward(qd, kd, vd, n)
    n.fill_(2000)
    g.replay()
    torch.cuda.synchronize()
    ref_new = ops.dense_attention(q.reshape(16, 128), k[0], v[0], 2000)
    ref_old = ops.dense_attention(q.reshape(16, 128), k[0], v[0], 1000)
    verdict = judge_length_change(correct_err=max_abs(out.cpu().reshape(16, 128), ref_new),
                                  stale_err=max_abs(ref_old, ref_new))
    assert verdict["verdict"] == "PASS", verdict


@pytest.mark.parametrize("ctx", [4096, 16384])
def test_attn_int8_vs_fp64_dequant(ctx, dev):
    from lemoq.kernels.attn_decode import attn_decode_forward_int8
    from lemoq.kernels.kv_int8 import kv_int8_bulk_quantize

    q, k, v = _qkv(16, ctx, 128, seed=ctx + 1)
    bufs = kv_int8_bulk_quantize(k.to(dev), v.to(dev))
    n = torch.tensor([ctx], dtype=torch.int32, device=dev)
    got = attn_decode_forward_int8(q.to(dev), bufs["kc"], bufs["ks"], bufs["vc"], bufs["vs"], n)
    kc, ks, vc, vs = (bufs[x][0].cpu() for x in ("kc", "ks", "vc", "vs"))
    ref64 = ops.int8_attention_dequant(q.reshape(16, 128), kc, ks, vc, vs, ctx)
    base = ops.int8_attention_folded(q.reshape(16, 128), kc, ks, vc, vs, ctx).to(torch.float16)
    assert_gate(got.cpu().reshape(16, 128), ref64, base, what="attn int8 ctx=%d" % ctx)


def test_attn_int8_partial_fill(dev):
    from lemoq.kernels.attn_decode import attn_decode_forward_int8
    from lemoq.kernels.kv_int8 import kv_int8_bulk_quantize

    q, k, v = _qkv(16, 512, 128, seed=91)
    bufs = kv_int8_bulk_quantize(k.to(dev), v.to(dev))
    for filled in (1, 33, 300):
        n = torch.tensor([filled], dtype=torch.int32, device=dev)
        got = attn_decode_forward_int8(q.to(dev), bufs["kc"], bufs["ks"], bufs["vc"], bufs["vs"], n)
        kc, ks, vc, vs = (bufs[x][0].cpu() for x in ("kc", "ks", "vc", "vs"))
        ref = ops.int8_attention_dequant(q.reshape(16, 128), kc, ks, vc, vs, filled)
        assert_close(got.cpu().reshape(16, 128), ref, rtol=1e-3, atol=1e-3, what="filled=%d" % filled)


# ---------------------------------------------------------------------------
# RMSNorm / RoPE
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,H", [(1, 2048), (16, 128), (3, 1000)])
def test_rmsnorm_vs_hf_formula(rows, H, dev):
    from lemoq.kernels.rmsnorm import rms_norm_fused

    x = randn(rows, H, seed=H).to(torch.float16)
    w = (torch.rand(H, generator=torch.Generator().manual_seed(H + 1)) + 0.5).to(torch.float16)
    got = rms_norm_fused(x.to(dev), w.to(dev), 1e-5).cpu()
    ref = ops.rms_norm(x, w, 1e-5)
    # fp16 rounding points are shared; the fp32 reduction order may move an element by 1 ulp
    assert_close(got, ref, rtol=1e-3, atol=1e-3, what="rmsnorm")
    assert (got.double() - ref.double()).abs().gt(0).float().mean() < 0.01


def test_rmsnorm_out_dtype_widens_the_fp16_result(dev):
    """out_dtype fp32: the same fp16 values in an fp32 buffer, as the reference
    stores its fp16 product into an out_dtype tensor (rmsnorm.py:147-160)."""
    from lemoq.kernels.rmsnorm import rms_norm_fused

    x = randn(4, 2048, seed=7).to(torch.float16).to(dev)
    w = (torch.rand(2048, generator=torch.Generator().manual_seed(8)) + 0.5).to(torch.float16).to(dev)
    y16 = rms_norm_fused(x, w, 1e-5)
    y32 = rms_norm_fused(x, w, 1e-5, out_dtype=torch.float32)
    assert y32.dtype == torch.float32 and torch.equal(y32, y16.float())


@pytest.mark.parametrize("rows,H,offset", [(3, 1003, 0), (4, 2048, 1), (2, 8192, 0)],
                         ids=["odd-width", "misaligned-rows", "widest"])
def test_rmsnorm_element_path_and_widest_rows(rows, H, offset, dev):
    """Rows that are not 16-byte chunks (odd width, or an input one element off
    alignment) take the per-element path; 8192-wide rows are the 16-byte path's
    widest.  Both against the oracle's RMSNorm."""
    from lemoq import _hip

    print("case: rmsnorm rows=%d H=%d offset=%d" % (rows, H, offset), flush=True)
    x = randn(rows, H, seed=H + offset).to(torch.float16)
    w = (torch.rand(H, generator=torch.Generator().manual_seed(H + 2)) + 0.5).to(torch.float16)
    xbuf = torch.zeros(rows * H + 8, dtype=torch.float16, device=dev)
    xd = xbuf[offset:offset + rows * H].view(rows, H)
    xd.copy_(x.to(dev))
    y = torch.empty((rows, H), dtype=torch.float16, device=dev)
    wd = w.to(dev)
    _hip.call("lemoq_rmsnorm", _hip.ptr(xd), rows, H, _hip.ptr(wd), 1e-5, _hip.ptr(y), _hip.stream_of(dev))
    got = y.cpu()
    ref = ops.rms_norm(x, w, 1e-5)
    assert_close(got, ref, rtol=1e-3, atol=1e-3, what="rmsnorm H=%d offset=%d" % (H, offset))
    assert (got.double() - ref.double()).abs().gt(0).float().mean() < 0.01


@pytest.mark.parametrize("pos", [0, 1, 1024, 4096])
def test_rope_fused_vs_oracle(pos, dev):
    from lemoq.kernels.rope import apply_rotary_pos_emb_fused, rotary_cos_sin

    q = randn(1, 16, 1, 128, seed=pos).to(torch.float16)
    k = randn(1, 16, 1, 128, seed=pos + 1).to(torch.float16)
    cos, sin = rotary_cos_sin([pos], 128)
    qo, ko = apply_rotary_pos_emb_fused(q.to(dev), k.to(dev), cos.reshape(1, 1, 128).to(dev),
                                        sin.reshape(1, 1, 128).to(dev))
    rq = ops.rope_fused(q, cos[0], sin[0])
    rk = ops.rope_fused(k, cos[0], sin[0])
    assert_close(qo.cpu(), rq, rtol=1e-3, atol=1e-3, what="rope q")
    assert_close(ko.cpu(), rk, rtol=1e-3, atol=1e-3, what="rope k")
    hq, hk = ops.rope_hf(q.float(), k.float(), cos[0].float(), sin[0].float())
    assert_close(qo.cpu(), hq, what="rope vs hf")


def test_rope_strided_views(dev):
    from lemoq.kernels.rope import apply_rotary_pos_emb_fused, rotary_cos_sin

    base = randn(1, 1, 16, 128, seed=5).to(torch.float16).to(dev)
    q = base.transpose(1, 2)  # (1,16,1,128) non-contiguous view
    k = base.transpose(1, 2)[:, :8]
    cos, sin = rotary_cos_sin([77], 128)
    qo, ko = apply_rotary_pos_emb_fused(q, k, cos.reshape(1, 1, 128).to(dev), sin.reshape(1, 1, 128).to(dev))
    rq = ops.rope_fused(q.cpu(), cos[0], sin[0])
    assert_close(qo.cpu(), rq, rtol=1e-3, atol=1e-3, what="strided rope")
    assert ko.shape == (1, 8, 1, 128)


def test_qk_norm_rope_kv_fused_prologue(dev):
    """The fused step prologue == rmsnorm -> rope -> per-token quant, codes bit-exact on its own k row."""
    from lemoq import _hip
    from lemoq.kernels.rope import rotary_cos_sin

    NH, D, S, pos = 16, 128, 64, 37
    HD = NH * D
    qkv = randn(3 * HD, seed=1).to(torch.float16)
    qn = (torch.rand(HD, generator=torch.Generator().manual_seed(2)) + 0.5).to(torch.float16)
    kn = (torch.rand(HD, generator=torch.Generator().manual_seed(3)) + 0.5).to(torch.float16)
    cos, sin = rotary_cos_sin(torch.arange(S), D)
    kc = torch.zeros((NH, S, D), dtype=torch.int8, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.ones((NH, S), dtype=torch.float16, device=dev)
    vs = torch.ones_like(ks)
    q_out = torch.empty(HD, dtype=torch.float16, device=dev)
    k_rot = torch.empty(HD, dtype=torch.float16, device=dev)
    kf = torch.zeros((NH, S, D), dtype=torch.float16, device=dev)
    vf = torch.zeros_like(kf)
    P = _hip.ptr
    # keep every device tensor referenced until the kernel has run
    qkv_d, qn_d, kn_d, cos_d, sin_d = (t.to(dev) for t in (qkv, qn, kn, cos, sin))
    pos_d = torch.tensor([pos], device=dev)
    _hip.call("lemoq_qk_norm_rope_kv_i8", P(qkv_d), NH, D, P(qn_d), P(kn_d), 1e-5, P(cos_d), P(sin_d),
              P(pos_d), P(q_out), P(kc), P(ks), P(vc), P(vs), S * D, S, P(kf), P(vf), S * D, P(k_rot),
              math.inf, _hip.stream_of(dev))
    torch.cuda.synchronize()
    q_ref = ops.rope_fused(ops.rms_norm(qkv[:HD], qn, 1e-5).reshape(NH, D), cos[pos], sin[pos])
    k_ref = ops.rope_fused(ops.rms_norm(qkv[HD:2 * HD], kn, 1e-5).reshape(NH, D), cos[pos], sin[pos])
    assert_close(q_out.cpu().reshape(NH, D), q_ref, rtol=1e-3, atol=1e-3, what="q")
    assert_close(k_rot.cpu().reshape(NH, D), k_ref, rtol=1e-3, atol=1e-3, what="k")
    rc, rs = oq.kv_quantize_rows(k_rot.cpu().reshape(NH, D).numpy())
    assert np.array_equal(kc[:, pos].cpu().numpy(), rc)
    assert np.array_equal(ks[:, pos].cpu().numpy().view(np.uint16), rs.view(np.uint16))
    vrc, vrs = oq.kv_quantize_rows(qkv[2 * HD:].reshape(NH, D).numpy())
    assert np.array_equal(vc[:, pos].cpu().numpy(), vrc)
    assert np.array_equal(vs[:, pos].cpu().numpy().view(np.uint16), vrs.view(np.uint16))
    assert torch.equal(kf[:, pos].cpu(), k_rot.cpu().reshape(NH, D))
    assert torch.equal(vf[:, pos].cpu(), qkv[2 * HD:].reshape(NH, D))
    other = torch.ones(S, dtype=torch.bool)
    other[pos] = False
    assert (kc[:, other] == 0).all() and (ks[:, other] == 1).all()


@pytest.mark.parametrize("ns", [1, 5, 16, 17, 64, 65, 200])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_attn_merge_vs_oracle(ns, D, dev):
    """lemoq_attn_merge (one wave per 64 dims up to 64 splits, the LDS kernel beyond)
    against the oracle's LSE merge: empty splits (m = -inf, l = 0, acc = 0), a head
    whose splits are all empty (-> 0), and m spread over 40 binades."""
    from lemoq import _hip

    heads = 3
    g = torch.Generator().manual_seed(ns * 1000 + D)
    m = (torch.rand((heads, ns), generator=g) * 40 - 20).float()
    l = torch.rand((heads, ns), generator=g).float() * 10 + 0.1
    acc = torch.randn((heads, ns, D), generator=g).float() * l.unsqueeze(-1)
    empty = torch.rand((heads, ns), generator=g) < 0.3
    empty[2] = True
    m[empty], l[empty], acc[empty] = float("-inf"), 0.0, 0.0
    out = torch.empty((heads * D,), dtype=torch.float16, device=dev)
    md, ld, ad = m.to(dev), l.to(dev), acc.to(dev)
    _hip.call("lemoq_attn_merge", _hip.ptr(md), _hip.ptr(ld), _hip.ptr(ad), heads, ns, D, _hip.ptr(out),
              _hip.stream_of(dev))
    ref = ops.merge_splits(m.double(), l.double(), acc.double())
    got = out.cpu().reshape(heads, D)
    assert torch.isfinite(got).all() and (got[2] == 0).all()
    assert_close(got, ref, what="merge ns=%d D=%d" % (ns, D))


def _merge_inputs(heads, ns, D, seed):
    g = torch.Generator().manual_seed(seed)
    m = (torch.rand((heads, ns), generator=g) * 40 - 20).float()
    l = torch.rand((heads, ns), generator=g).float() * 10 + 0.1
    acc = torch.randn((heads, ns, D), generator=g).float() * l.unsqueeze(-1)
    empty = torch.rand((heads, ns), generator=g) < 0.3
    empty[1] = True  # one head with every split empty -> attention output 0
    m[empty], l[empty], acc[empty] = float("-inf"), 0.0, 0.0
    return m, l, acc


@pytest.mark.parametrize("ns", [1, 5, 16, 17, 64])
@pytest.mark.parametrize("heads", [16, 4, 8, 32])
@pytest.mark.parametrize("bits", [8, 4])
def test_merge_o_proj_partials(ns, heads, bits, dev):
    """lemoq_attn_merge_o_proj_w8 / _w4 (merge fused into o_proj, split over
    groups of 4 heads; int8 or packed 4-bit codes).  Its merge is
    lemoq_attn_merge's, so each partial row g must equal the fp64 product of the
    dequantised columns [512g, 512g+512) with the merged fp16 attention output of
    lemoq_attn_merge, to fp32 summation error; fp16(sum of partials) is the
    o_proj output (oracle: LSE merge in fp64, then the linear)."""
    from lemoq import _hip

    D, N, group = 128, 2048, 128
    HD = heads * D
    m, l, acc = _merge_inputs(heads, ns, D, seed=ns * 7 + heads)
    w = randn(N, HD, seed=900 + heads, std=0.02)
    if bits == 8:
        codes, scale = _q8(w, group)
        stored = codes
    else:
        q = oq.rtn_quantize(w.numpy(), bits=4, group_size=group, symmetric=True)
        codes = torch.from_numpy(q["codes_padded"].astype(np.int8))  # unpacked, for the oracle
        stored, scale = torch.from_numpy(oq.pack_4bit(q["codes_padded"])), torch.from_numpy(q["scale_f16"])
    md, ld, ad, cd, sd = (t.to(dev) for t in (m, l, acc, stored, scale))
    part = torch.full((heads // 4, N), float("nan"), dtype=torch.float32, device=dev)
    attn = torch.empty((HD,), dtype=torch.float16, device=dev)
    st = _hip.stream_of(dev)
    _hip.call("lemoq_attn_merge_o_proj_w%d" % bits, _hip.ptr(md), _hip.ptr(ld), _hip.ptr(ad), heads, ns, D,
              _hip.ptr(cd), _hip.ptr(sd), N, group, _hip.ptr(part), st)
    _hip.call("lemoq_attn_merge", _hip.ptr(md), _hip.ptr(ld), _hip.ptr(ad), heads, ns, D, _hip.ptr(attn), st)
    torch.cuda.synchronize()
    p = part.cpu().double()
    assert torch.isfinite(p).all()
    wd = ops.dequant_w8(codes, scale, group).double()  # (N, HD), the fp16-rounded weights
    a = attn.cpu().double()
    for gi in range(heads // 4):
        cols = slice(512 * gi, 512 * gi + 512)
        ref = wd[:, cols] @ a[cols]
        err = (p[gi] - ref).abs().max().item()
        assert err <= 1e-5 * (wd[:, cols].abs() @ a[cols].abs()).max().item() + 1e-7, (gi, err)
    got = p.sum(0).to(torch.float16)
    a_ref = ops.merge_splits(m.double(), l.double(), acc.double()).reshape(-1).to(torch.float16)
    ref = ops.dequant_gemm_separate(a_ref.reshape(1, -1), codes, scale, group).reshape(-1)
    assert_close(got, ref, what="merge+o_proj ns=%d heads=%d" % (ns, heads))


@pytest.mark.parametrize("H,n_part", [(2048, 4), (2048, 1), (2048, 2), (2048, 8), (4096, 4)])
@pytest.mark.parametrize("E", [64, 8, 100])
def test_router_logits_resid_vs_oracle(H, n_part, E, dev):
    """lemoq_router_logits_resid: h' = fp16(fp16(sum of partials) + h) must be
    bit-exact against the same fp32 sum and fp16 add on the CPU; xn and the
    logits against the oracle's RMSNorm and router linear (the bounds of the
    lemoq_router_logits test), and the routing of the logits must give the
    oracle's expert ids."""
    from lemoq import _hip

    gen = torch.Generator().manual_seed(H + n_part * 10 + E)
    part = torch.randn((n_part, H), generator=gen).float() * 0.5
    h = randn(H, seed=E + 1).to(torch.float16)
    ln = (torch.rand(H, generator=gen) + 0.5).to(torch.float16)
    rw = randn(E, H, seed=E + 2, std=0.02).to(torch.float16)
    pd, hd, lnd, rwd = part.to(dev), h.to(dev), ln.to(dev), rw.to(dev)
    h_out = torch.empty(H, dtype=torch.float16, device=dev)
    xn = torch.empty(H, dtype=torch.float16, device=dev)
    lg = torch.empty(E, dtype=torch.float16, device=dev)
    _hip.call("lemoq_router_logits_resid", _hip.ptr(pd), n_part, _hip.ptr(hd), _hip.ptr(lnd), 1e-5, H,
              _hip.ptr(rwd), E, _hip.ptr(h_out), _hip.ptr(xn), _hip.ptr(lg), _hip.stream_of(dev))
    torch.cuda.synchronize()
    o = part[0].clone()
    for gi in range(1, n_part):
        o = o + part[gi]  # fp32, group order
    h_mid = o.to(torch.float16) + h  # torch's fp16 add: one rounding
    assert torch.equal(h_out.cpu(), h_mid)
    xn_ref = ops.rms_norm(h_mid, ln, 1e-5)
    assert max_abs(xn.cpu(), xn_ref) <= 2e-3
    rlg, _, rti = ops.route(xn_ref.reshape(1, H), rw, min(8, E), True)
    assert max_abs(lg.cpu(), rlg.reshape(-1)) <= 2e-3
    # the step's other router on h' gives the same fp16 outputs
    xn2 = torch.empty_like(xn)
    lg2 = torch.empty_like(lg)
    hm = h_mid.to(dev)
    _hip.call("lemoq_router_logits", _hip.ptr(hm), _hip.ptr(lnd), 1e-5, H, _hip.ptr(rwd), E, _hip.ptr(xn2),
              _hip.ptr(lg2), _hip.stream_of(dev))
    torch.cuda.synchronize()
    assert max_abs(xn.cpu(), xn2.cpu()) <= 2e-3 and max_abs(lg.cpu(), lg2.cpu()) <= 2e-3


def _advance(hip, dev, logits, pos, prompt=None, history_len=64):
    """One lemoq_argmax_advance; returns (token, pos, filled, history)."""
    ld = logits.to(dev)
    tok = torch.full((1,), -7, dtype=torch.int64, device=dev)
    pd = torch.tensor([pos], dtype=torch.int64, device=dev)
    fd = torch.zeros((1,), dtype=torch.int32, device=dev)
    hist = torch.full((history_len,), -5, dtype=torch.int64, device=dev)
    pr = torch.tensor(prompt, dtype=torch.int64, device=dev) if prompt is not None else None
    hip.call("lemoq_argmax_advance", hip.ptr(ld), logits.numel(), hip.ptr(tok), hip.ptr(pd), hip.ptr(fd),
             hip.ptr(pr) if pr is not None else None, len(prompt) if prompt is not None else 0, hip.ptr(hist),
             history_len, hip.stream_of(dev))
    torch.cuda.synchronize()
    return int(tok.item()), int(pd.item()), int(fd.item()), hist.cpu()


def _first_argmax(x: torch.Tensor) -> int:
    """Lowest index of the largest non-NaN value (0 when there is none)."""
    v = x.float().clone()
    v[torch.isnan(v)] = float("-inf")
    m = v.max()
    return int(torch.nonzero(v == m)[0]) if m > float("-inf") or (v == m).any() else 0


@pytest.mark.parametrize("n", [1, 5, 1023, 8192, 8195, 50304])
def test_argmax_advance_ties_nan_and_passes(n, dev):
    """Greedy selection of lemoq_argmax_advance (the device form of the
    reference's logits.argmax(), cudagraph.py:759-762): lowest index on ties,
    NaN never selected, all -inf -> 0; n spans one and several passes of
    8 x 1024 candidates."""
    from lemoq import _hip

    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, generator=g).to(torch.float16)
    tok, p, f, hist = _advance(_hip, dev, x, 9)
    assert tok == _first_argmax(x) and p == 10 and f == 11 and int(hist[10]) == tok
    if n >= 5:
        y = x.clone()
        top = float(y.float().max()) + 1.0
        y[n - 1] = top
        y[n // 2] = top
        y[1] = float("nan")
        tok, _, _, _ = _advance(_hip, dev, y, 0)
        assert tok == n // 2 if n // 2 < n - 1 else tok == n - 1
        assert tok == _first_argmax(y)
    z = torch.full((n,), float("-inf"), dtype=torch.float16)
    assert _advance(_hip, dev, z, 0)[0] == 0
    z[n - 1] = float("nan")
    assert _advance(_hip, dev, z, 0)[0] == 0
    if n >= 3:
        z[n - 2] = -60000.0
        assert _advance(_hip, dev, z, 0)[0] == n - 2


def test_argmax_advance_prompt_feed_and_history_bounds(dev):
    """While pos + 1 < prompt_len the next token is prompt[pos + 1], after that
    the argmax; history[pos + 1] is written only inside history_len."""
    from lemoq import _hip

    x = torch.zeros(100, dtype=torch.float16)
    x[42] = 3.0
    prompt = [11, 12, 13, 14]
    assert _advance(_hip, dev, x, 0, prompt)[0] == 12
    assert _advance(_hip, dev, x, 2, prompt)[0] == 14
    assert _advance(_hip, dev, x, 3, prompt)[0] == 42
    tok, p, f, hist = _advance(_hip, dev, x, 7, history_len=8)  # pos + 1 == history_len: no write
    assert tok == 42 and p == 8 and f == 9 and (hist == -5).all()


@pytest.mark.parametrize("N", [50304, 1000, 37])
def test_lm_head_argmax_partials(N, dev):
    """lemoq_lm_head_argmax_w8: the fp16 logits of the w8 GEMV (final RMSNorm in
    the prologue) against the oracle, and the selected token equal to the
    lowest-index argmax of the GPU's own logits (the partial reduction must not
    change the selection)."""
    from lemoq import _hip

    H, group = 2048, 128
    w = randn(N, H, seed=N, std=0.02)
    codes, scale = _q8(w, group)
    x = randn(H, seed=N + 1).to(torch.float16)
    nw = (torch.rand(H, generator=torch.Generator().manual_seed(N)) + 0.5).to(torch.float16)
    xd, nd, cd, sd = x.to(dev), nw.to(dev), codes.to(dev), scale.to(dev)
    parts = int(_hip.load().lemoq_lm_head_argmax_parts(N))
    pv = torch.empty(parts, dtype=torch.float32, device=dev)
    pi = torch.empty(parts, dtype=torch.int32, device=dev)
    logits = torch.empty(N, dtype=torch.float16, device=dev)
    tok = torch.zeros(1, dtype=torch.int64, device=dev)
    pos = torch.zeros(1, dtype=torch.int64, device=dev)
    fill = torch.zeros(1, dtype=torch.int32, device=dev)
    _hip.call("lemoq_lm_head_argmax_w8", _hip.ptr(xd), _hip.ptr(nd), 1e-5, _hip.ptr(cd), _hip.ptr(sd), N, H, group,
              _hip.ptr(logits), _hip.ptr(pv), _hip.ptr(pi), parts, _hip.ptr(tok), _hip.ptr(pos), _hip.ptr(fill),
              None, 0, None, 0, _hip.stream_of(dev))
    torch.cuda.synchronize()
    lg = logits.cpu()
    ref = ops.dequant_gemm_separate(ops.rms_norm(x, nw, 1e-5).reshape(1, -1), codes, scale, group).reshape(-1)
    assert_close(lg, ref, what="lm_head N=%d" % N)
    assert int(tok.item()) == _first_argmax(lg)
    assert int(pos.item()) == 1 and int(fill.item()) == 2


@pytest.mark.parametrize("N", [50304, 1000, 37])
def test_lm_head_argmax_dequant_first(N, dev):
    """lemoq_lm_head_argmax_w8_dq (the prefill's last row): the weights rounded to
    fp16(code * scale) before the dot, as the separate arm's F.linear over the
    dequantised lm_head.  Logits within one fp16 step of the fp64 product with those
    fp16 weights (plus fp32 accumulation), the token the lowest-index argmax of the
    GPU's logits, and the step advanced as lemoq_argmax_advance does."""
    from lemoq import _hip

    H, group = 2048, 128
    w = randn(N, H, seed=N + 5, std=0.02)
    codes, scale = _q8(w, group)
    x = randn(H, seed=N + 6).to(torch.float16)
    nw = (torch.rand(H, generator=torch.Generator().manual_seed(N + 7)) + 0.5).to(torch.float16)
    xd, nd, cd, sd = x.to(dev), nw.to(dev), codes.to(dev), scale.to(dev)
    parts = int(_hip.load().lemoq_lm_head_argmax_parts(N))
    pv = torch.empty(parts, dtype=torch.float32, device=dev)
    pi = torch.empty(parts, dtype=torch.int32, device=dev)
    logits = torch.empty(N, dtype=torch.float16, device=dev)
    tok = torch.zeros(1, dtype=torch.int64, device=dev)
    pos = torch.full((1,), 4, dtype=torch.int64, device=dev)
    fill = torch.zeros(1, dtype=torch.int32, device=dev)
    hist = torch.full((8,), -5, dtype=torch.int64, device=dev)
    prompt = torch.arange(5, dtype=torch.int64, device=dev)
    _hip.call("lemoq_lm_head_argmax_w8_dq", _hip.ptr(xd), _hip.ptr(nd), 1e-5, _hip.ptr(cd), _hip.ptr(sd), N, H,
              group, _hip.ptr(logits), _hip.ptr(pv), _hip.ptr(pi), parts, _hip.ptr(tok), _hip.ptr(pos),
              _hip.ptr(fill), _hip.ptr(prompt), 5, _hip.ptr(hist), 8, _hip.stream_of(dev))
    torch.cuda.synchronize()
    lg = logits.cpu()
    xn = ops.rms_norm(x, nw, 1e-5)
    ref = ops.dequant_gemm_separate(xn.reshape(1, -1), codes, scale, group).reshape(-1)
    assert_close(lg, ref, what="lm_head dq N=%d" % N)
    w16 = (codes.float() * scale.float().repeat_interleave(group, dim=1)).to(torch.float16)
    exact = (w16.double() @ xn.double()).reshape(-1)
    ulp = torch.finfo(torch.float16).eps * exact.abs().clamp_min(2.0 ** -14)
    allow = ulp + 3e-5 * (w16.double().abs() @ xn.double().abs()).reshape(-1)
    assert bool(((lg.double() - exact).abs() <= allow).all()), "dq logits beyond one fp16 step"
    assert int(tok.item()) == _first_argmax(lg)
    assert int(pos.item()) == 5 and int(fill.item()) == 6
    assert int(hist[5].item()) == int(tok.item())


@pytest.mark.parametrize("N,H", [(50304, 2048), (1000, 2048), (37, 2048), (203, 1040)])
def test_lm_head_argmax_f16(N, H, dev):
    """lemoq_lm_head_argmax_f16 (the fp16 lm_head of the w4a16 cell): logits
    bit-identical to lemoq_router_logits over the same rows (same lane order and
    butterfly), within one fp16 step of the oracle's fp64 F.linear of the normed
    row, the token the lowest-index argmax of those logits (a tie planted across
    blocks: two identical winning rows), and the step advanced as
    lemoq_argmax_advance does (prompt feed, history write)."""
    from lemoq import _hip

    w = randn(N, H, seed=N + 11, std=0.02)
    x = randn(H, seed=N + 12).to(torch.float16)
    nw = (torch.rand(H, generator=torch.Generator().manual_seed(N + 13)) + 0.5).to(torch.float16)
    xn = ops.rms_norm(x, nw, 1e-5)
    a, b = 3, N - 2  # different blocks (8 rows each) at every N here
    w[a] = w[b] = 0.05 * torch.sign(xn.float())
    w16 = w.to(torch.float16)
    xd, nd, wd = x.to(dev), nw.to(dev), w16.to(dev)
    parts = int(_hip.load().lemoq_lm_head_argmax_parts(N))
    pv = torch.empty(parts, dtype=torch.float32, device=dev)
    pi = torch.empty(parts, dtype=torch.int32, device=dev)
    logits = torch.empty(N, dtype=torch.float16, device=dev)
    ref_logits = torch.empty(N, dtype=torch.float16, device=dev)
    tok = torch.zeros(1, dtype=torch.int64, device=dev)
    fill = torch.zeros(1, dtype=torch.int32, device=dev)
    hist = torch.full((8,), -5, dtype=torch.int64, device=dev)
    prompt = torch.arange(100, 105, dtype=torch.int64, device=dev)
    st = _hip.stream_of(dev)
    toks = []
    for p0 in (2, 4):  # inside the prompt (fed), then past it (argmax)
        pos = torch.full((1,), p0, dtype=torch.int64, device=dev)
        _hip.call("lemoq_lm_head_argmax_f16", _hip.ptr(xd), _hip.ptr(nd), 1e-5, _hip.ptr(wd), N, H, _hip.ptr(logits),
                  _hip.ptr(pv), _hip.ptr(pi), parts, _hip.ptr(tok), _hip.ptr(pos), _hip.ptr(fill), _hip.ptr(prompt), 5,
                  _hip.ptr(hist), 8, st)
        torch.cuda.synchronize()
        toks.append(int(tok.item()))
        assert int(pos.item()) == p0 + 1 and int(fill.item()) == p0 + 2
        assert int(hist[p0 + 1].item()) == toks[-1]
    _hip.call("lemoq_router_logits", _hip.ptr(xd), _hip.ptr(nd), 1e-5, H, _hip.ptr(wd), N, None,
              _hip.ptr(ref_logits), st)
    torch.cuda.synchronize()
    lg = logits.cpu()
    assert torch.equal(lg.view(torch.int16), ref_logits.cpu().view(torch.int16)), "not the router kernel's logits"
    exact = (w16.double() @ xn.double()).reshape(-1)
    ulp = torch.finfo(torch.float16).eps * exact.abs().clamp_min(2.0 ** -14)
    allow = ulp + 3e-5 * (w16.double().abs() @ xn.double().abs()).reshape(-1)
    assert bool(((lg.double() - exact).abs() <= allow).all()), "fp16 lm_head logits beyond one fp16 step"
    assert toks[0] == 103  # prompt[pos + 1] while pos + 1 < prompt_len
    assert lg[a] == lg[b] and _first_argmax(lg) == a and toks[1] == a


def test_warm_entry_points_run_before_capture(dev):
    """The reference's warm() hooks (one real launch, then sync) exist with the
    same signatures and run on the device."""
    from lemoq.kernels import attn_decode, dequant_gemm, rmsnorm, rope

    rope.warm(device=dev)
    rope.warm(heads=16, kv_heads=16, head_dim=128, device=dev)
    x = randn(1, 2048, seed=70).to(torch.float16).to(dev)
    rmsnorm.warm(x, torch.ones(2048, dtype=torch.float16, device=dev), 1e-5)
    codes, scale = _q8(randn(256, 2048, seed=71, std=0.02), 128)
    dequant_gemm.warm(x, codes.to(dev), scale.to(dev), None, group_size=128, bits=8)
    attn_decode.warm(heads=16, head_dim=128, kv_len=512, device=dev)
