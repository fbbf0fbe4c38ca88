"""GPU parity of the multi-token linears on the matrix cores.

``lemoq_gemm_w8`` follows the reference's multi-token ``QuantLinear`` arm
(fp16 dequantised weight, ``F.linear``: src/lemoq/quant/linear.py:365-395,
471-480) and ``lemoq_gemm_f16`` the router's fp16 ``F.linear`` for several
tokens (src/lemoq/kernels/moe_static.py:267).  The oracle forms each product
in fp64 from the same fp16 weight and rounds once to fp16; the kernel
accumulates in fp32, so every output lies within one fp16 ulp of the oracle
plus an fp32 accumulation allowance of 3e-5 * sum|x||w| (the worst case for
K = 2048 is 2048 * 2^-24 = 1.2e-4; observed errors are far below the
allowance).  The fp16 output tolerance of the decode-step target (rtol 2e-2, atol 2e-3) is checked as well.
Shapes: the OLMoE prefill linears (qkv 6144 x 2048, o_proj 2048 x 2048, one
expert's gate_up 2048 x 2048 and down 2048 x 1024, router 64 x 2048, lm_head
50304 x 2048 for the last row), ragged M and N, row gather and residual.
"""

from __future__ import annotations

import pytest
import torch

from helpers import assert_close, randn
from oracle import ops
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def _q8(w: torch.Tensor, group: int):
    q = oq.rtn_quantize_w8(w.numpy(), group)
    return torch.from_numpy(q["codes_padded"]), torch.from_numpy(q["scale_f16"])


def _ulp16(r: torch.Tensor) -> torch.Tensor:
    a = r.double().abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


def _assert_linear(got, ref16, absdot, what):
    g, r = got.double().cpu(), ref16.double()
    assert g.shape == r.shape, what
    assert torch.isfinite(g).all(), what
    bound = _ulp16(r) + 3e-5 * absdot
    err = (g - r).abs()
    assert bool((err <= bound).all()), "%s: max err %.3e, worst excess %.3e" % (
        what, float(err.max()), float((err - bound).max()))
    assert_close(got, ref16, what=what)


SHAPES = [
    (2, 384, 256),       # tiny
    (16, 6144, 2048),    # qkv, short prompt
    (100, 2048, 2048),   # o_proj, ragged M
    (1024, 6144, 2048),  # qkv at ctx 1024
    (37, 100, 128),      # ragged M and N, one group
    (257, 2048, 1024),   # expert down width
    (1, 50304, 2048),    # lm_head on the last prompt row
    (2000, 2048, 256),   # 128 x 128 tiles of 8 waves (>= 256 of them, < 192 of 256 x 128), ragged M
    (1100, 6100, 512),   # 256 x 128 tiles of 8 waves, ragged M and N
]


@pytest.mark.parametrize("m,n,k", SHAPES, ids=["%dx%dx%d" % s for s in SHAPES])
def test_gemm_w8_vs_oracle(m, n, k, dev):
    from lemoq.kernels.dequant_gemm import dequant_gemm_separate

    print("case: gemm_w8 m=%d n=%d k=%d" % (m, n, k), flush=True)
    codes, scale = _q8(randn(n, k, seed=n + k, std=0.02), 128)
    x = randn(m, k, seed=3 * m + k).to(torch.float16)
    got = dequant_gemm_separate(x.to(dev), codes.to(dev), scale.to(dev), group_size=128)
    torch.cuda.synchronize()
    ref = ops.linear_separate_w8(x, codes, scale, 128)
    absdot = x.double().abs() @ ops.dequant_weight_f16(codes, scale, 128).double().abs().t()
    _assert_linear(got, ref, absdot, "gemm_w8 %dx%dx%d" % (m, n, k))


def test_gemm_w8_gather_and_residual(dev):
    from lemoq import _hip

    print("case: gemm_w8 gather + residual", flush=True)
    rows, m, n, k = 300, 77, 512, 1024
    codes, scale = _q8(randn(n, k, seed=41, std=0.02), 128)
    x = randn(rows, k, seed=42).to(torch.float16)
    idx = torch.randint(0, rows, (m,), generator=torch.Generator().manual_seed(43), dtype=torch.int32)
    resid = randn(m, n, seed=44).to(torch.float16)
    xd, cd, sd, idd = x.to(dev), codes.to(dev), scale.to(dev), idx.to(dev)
    y = resid.clone().to(dev)  # residual aliases the output
    _hip.call("lemoq_gemm_w8", _hip.ptr(xd), m, k, k, _hip.ptr(idd), _hip.ptr(cd), _hip.ptr(sd), n, 128,
              _hip.ptr(y), n, _hip.ptr(y), n, _hip.stream_of(dev))
    torch.cuda.synchronize()
    xg = x[idx.long()]
    lin = ops.linear_separate_w8(xg, codes, scale, 128)
    ref = (lin.float() + resid.float()).to(torch.float16)
    absdot = xg.double().abs() @ ops.dequant_weight_f16(codes, scale, 128).double().abs().t()
    # one ulp of the linear output can move the sum by one more rounding step
    err = (y.cpu().double() - ref.double()).abs()
    bound = _ulp16(ref) + _ulp16(lin) + 3e-5 * absdot
    assert bool((err <= bound).all()), float((err - bound).max())
    assert_close(y.cpu(), ref, what="gather+residual")


@pytest.mark.parametrize("m,n,k", [(1100, 6144, 256), (2000, 2048, 256), (77, 512, 1024)],
                         ids=["256x128-tiles", "128x128-tiles", "64x64-tiles"])
def test_gemm_w8_row_stores_equal_element_stores(m, n, k, dev):
    """16-byte aligned output rows are staged in LDS and written as 16-byte
    chunks; an output one element off that alignment takes the per-element
    stores.  Both give the same bytes, with and without the residual, into a
    strided output (y_ld > N) whose pad columns stay untouched."""
    from lemoq import _hip

    print("case: gemm_w8 row vs element stores m=%d n=%d k=%d" % (m, n, k), flush=True)
    codes, scale = _q8(randn(n, k, seed=51, std=0.02), 128)
    x = randn(m, k, seed=52).to(torch.float16)
    resid = randn(m, n, seed=53).to(torch.float16)
    xd, cd, sd = x.to(dev), codes.to(dev), scale.to(dev)
    P, st = _hip.ptr, _hip.stream_of(dev)
    ld = n + 8
    outs = {}
    for off in (0, 1):  # 0: 16-byte aligned rows; 1: one fp16 element off
        for with_resid in (False, True):
            buf = torch.full((m * ld + 16,), float("nan"), dtype=torch.float16, device=dev)
            y = buf[off:off + m * ld].view(m, ld)
            rbuf = torch.zeros((m * ld + 16,), dtype=torch.float16, device=dev)
            r = rbuf[off:off + m * ld].view(m, ld)
            r[:, :n] = resid.to(dev)
            _hip.call("lemoq_gemm_w8", P(xd), m, k, k, None, P(cd), P(sd), n, 128, P(y), ld,
                      P(r) if with_resid else None, ld, st)
            torch.cuda.synchronize()
            assert bool(torch.isnan(y[:, n:]).all()), "pad columns written"
            outs[(off, with_resid)] = y[:, :n].cpu()
    for with_resid in (False, True):
        assert torch.equal(outs[(0, with_resid)], outs[(1, with_resid)]), with_resid
    ref = ops.linear_separate_w8(x, codes, scale, 128)
    assert_close(outs[(0, False)], ref, what="row stores vs oracle")
    assert_close(outs[(0, True)], (ref.float() + resid.float()).to(torch.float16), what="row stores + residual")


@pytest.mark.parametrize("m,n,k", [(1024, 64, 2048), (5, 64, 2048), (3, 50, 64)])
def test_gemm_f16_vs_oracle(m, n, k, dev):
    from lemoq.kernels.dequant_gemm import linear_f16

    print("case: gemm_f16 m=%d n=%d k=%d" % (m, n, k), flush=True)
    w = randn(n, k, seed=n * k, std=0.02).to(torch.float16)
    x = randn(m, k, seed=m + 5).to(torch.float16)
    got = linear_f16(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    ref = ops.linear_f16(x, w)
    _assert_linear(got, ref, x.double().abs() @ w.double().abs().t(), "gemm_f16 %dx%dx%d" % (m, n, k))


@pytest.mark.parametrize("m,n,k,splits", [(1024, 64, 2048, 8), (5, 64, 2048, 4), (3, 50, 128, 2), (70, 64, 2048, 1)])
def test_gemm_f16_splitk_vs_oracle(m, n, k, splits, dev):
    from lemoq.kernels.dequant_gemm import linear_f16

    print("case: gemm_f16 split-K m=%d n=%d k=%d splits=%d" % (m, n, k, splits), flush=True)
    w = randn(n, k, seed=n + k + splits, std=0.02).to(torch.float16)
    x = randn(m, k, seed=m + 9).to(torch.float16)
    got = linear_f16(x.to(dev), w.to(dev), splits=splits)
    torch.cuda.synchronize()
    ref = ops.linear_f16(x, w)
    _assert_linear(got, ref, x.double().abs() @ w.double().abs().t(), "gemm_f16 split %d" % splits)


def test_quant_linear_dispatch(dev):
    """One row takes the fused GEMV, several rows the separate-arm GEMM (as the reference's forward)."""
    from lemoq.kernels.dequant_gemm import dequant_gemm_fused, dequant_gemm_separate
    from lemoq.quant.linear import QuantLinear

    print("case: QuantLinear dispatch", flush=True)
    lin = QuantLinear(randn(1024, 2048, seed=61, std=0.02).to(dev))
    x1 = randn(1, 2048, seed=62).to(torch.float16).to(dev)
    x7 = randn(1, 7, 2048, seed=63).to(torch.float16).to(dev)
    assert torch.equal(lin(x1), dequant_gemm_fused(x1, lin.packed, lin.scale, None, group_size=128,
                                                   out_dtype=torch.float16))
    y7 = lin(x7)
    assert y7.shape == (1, 7, 1024)
    assert torch.equal(y7.reshape(7, 1024), dequant_gemm_separate(x7.reshape(7, 2048), lin.packed, lin.scale,
                                                                  group_size=128))


def test_gemm_f16_splitk_one_split_ignores_the_workspace(dev):
    """splits == 1 is lemoq_gemm_f16: a workspace passed anyway must stay unused and y must be written."""
    from lemoq import _hip

    print("case: gemm_f16 split-K with one split and a workspace", flush=True)
    m, n, k = 5, 64, 512
    w = randn(n, k, seed=77, std=0.05).to(torch.float16)
    x = randn(m, k, seed=78).to(torch.float16)
    ws = torch.full((1, m, n), float("nan"), dtype=torch.float32, device=dev)
    y = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    y1 = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    xd, wd = x.to(dev), w.to(dev)
    P, st = _hip.ptr, _hip.stream_of(dev)
    _hip.call("lemoq_gemm_f16_splitk", P(xd), m, k, k, P(wd), n, P(y), n, 1, P(ws), st)
    _hip.call("lemoq_gemm_f16", P(xd), m, k, k, P(wd), n, P(y1), n, st)
    torch.cuda.synchronize()
    assert torch.isnan(ws).all()
    assert torch.equal(y.cpu().view(torch.int16), y1.cpu().view(torch.int16))
    _assert_linear(y, ops.linear_f16(x, w), x.double().abs() @ w.double().abs().t(), "gemm_f16 split 1")


@pytest.mark.parametrize("m,n,k,splits,top_k,norm", [(1000, 64, 2048, 8, 8, False), (37, 64, 2048, 4, 8, True),
                                                     (1, 16, 256, 2, 4, False), (300, 128, 4096, 8, 8, True),
                                                     (50, 64, 3072, 12, 8, False)])
def test_route_topk_of_splitk_partials(m, n, k, splits, top_k, norm, dev):
    """The router's partials-only split-K GEMM followed by the routing that sums them gives the
    same ids and weights, bit for bit, as the GEMM's own finish followed by lemoq_route_topk, and
    the oracle's routing of the oracle's logits."""
    from lemoq import _hip

    print("case: route_topk_splitk m=%d n=%d k=%d splits=%d" % (m, n, k, splits), flush=True)
    w = randn(n, k, seed=3 * n + k, std=0.05).to(torch.float16)
    x = randn(m, k, seed=m + 11).to(torch.float16)
    xd, wd = x.to(dev), w.to(dev)
    P, st = _hip.ptr, _hip.stream_of(dev)
    ws = torch.full((splits, m, n), float("nan"), dtype=torch.float32, device=dev)
    logits = torch.empty((m, n), dtype=torch.float16, device=dev)
    tw = [torch.empty((m, top_k), dtype=torch.float32, device=dev) for _ in range(2)]
    ti = [torch.full((m, top_k), -1, dtype=torch.int64, device=dev) for _ in range(2)]
    _hip.call("lemoq_gemm_f16_splitk", P(xd), m, k, k, P(wd), n, P(logits), n, splits, P(ws), st)
    _hip.call("lemoq_route_topk", P(logits), 1, m, n, n, top_k, int(norm), P(tw[0]), P(ti[0]), st)
    ws.fill_(float("nan"))
    _hip.call("lemoq_gemm_f16_splitk", P(xd), m, k, k, P(wd), n, None, n, splits, P(ws), st)
    _hip.call("lemoq_route_topk_splitk", P(ws), splits, m, n, top_k, int(norm), P(tw[1]), P(ti[1]), st)
    torch.cuda.synchronize()
    assert not torch.isnan(ws).any()  # every partial was written by the partials-only launch
    assert torch.equal(ti[0].cpu(), ti[1].cpu())
    assert torch.equal(tw[0].cpu(), tw[1].cpu())
    # 1. Given the same logits the routing is exact: the oracle's routing of the
    #    GPU's own fp16 logits selects the same ids, in the same order, on every row.
    got16 = logits.cpu()
    rw_g, ri_g = ops.route_logits(got16, top_k, norm)
    assert torch.equal(ri_g, ti[0].cpu()), "routing of identical logits differs"
    torch.testing.assert_close(tw[0].cpu(), rw_g, rtol=1e-5, atol=1e-6)
    # 2. Against the oracle's own logits (the fp64 product rounded once), the
    #    GPU's fp32-accumulated logits may sit one fp16 step away.  A row may then
    #    route differently only where two of the oracle's first top_k + 1 logits
    #    (sorted) are within that measured logit error of each other; every
    #    other row must select exactly the oracle's ids.
    ref16 = ops.linear_f16(x, w)
    rw, ri = ops.route_logits(ref16, top_k, norm)
    err = float((got16.double() - ref16.double()).abs().max())
    srt = torch.sort(ref16.double(), dim=-1, descending=True).values[:, : top_k + 1]
    close = (srt[:, :-1] - srt[:, 1:]).min(dim=-1).values <= err
    same = (ri == ti[1].cpu()).all(dim=-1)
    excused = int((~same & close).sum())
    print("rows %d, logit error %.2e, rows with a gap <= error %d, excused id differences %d"
          % (m, err, int(close.sum()), excused))
    assert bool((same | close).all()), "ids differ on a row with no near-tie: %s" % (
        torch.nonzero(~(same | close)).flatten()[:8].tolist())
    torch.testing.assert_close(tw[1].cpu()[same], rw[same], rtol=2e-2, atol=2e-3)
