"""RMSNorm rounding points on the GPU, bit for bit against the oracle.

The reference's RMSNorm (HF ``OlmoeRMSNorm``, the fused kernel's contract
``src/lemoq/kernels/rmsnorm.py:184-202``, restated by ``oracle.ops.rms_norm``)
computes ``x * rsqrt(mean(x^2) + eps)`` in fp32, rounds that fp32 value to
fp16, and multiplies by the fp16 weight in fp16.  A kernel whose compiler
folds the fp32 multiply into the conversion (one mixed-precision op that
rounds the exact product straight to fp16) differs wherever the fp32 rounding
lands on an fp16 tie.

The rows here hold values k / 64 with |k| <= 88: their squares sum exactly in
fp32 in any order, so every implementation's sum, mean and rstd are the same
fp32 numbers and the normalised rows must match the oracle exactly (the other
RMSNorm tests allow an ulp for the reduction order).  The inputs are checked
to contain elements where the two roundings differ, so a single-rounding
kernel cannot pass.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lemoq import _hip
from oracle import ops

pytestmark = pytest.mark.gpu

EPS = 1e-5


def _rows(rows: int, H: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    k = torch.randint(-88, 89, (rows, H), generator=g)
    x = (k.double() / 64).half()
    w = (torch.rand(H, generator=g) + 0.5).half()
    return x, w


def _single_rounding_differs(x: torch.Tensor) -> int:
    """Elements where rounding the exact product x * rstd once to fp16 differs
    from rounding it to fp32 first (the sensitivity of these inputs)."""
    xf = x.float()
    rstd = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)
    dbl = (xf * rstd).half()
    sgl = torch.from_numpy((x.double() * rstd.double()).numpy().astype(np.float16))
    return int((dbl.view(torch.int16) != sgl.view(torch.int16)).sum())


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().cpu().contiguous().view(torch.int16)


def test_inputs_sum_exactly_and_are_sensitive():
    x, _ = _rows(1024, 2048, 0)
    sq = x.float().pow(2)
    assert torch.equal(sq.sum(-1), sq.flip(-1).cumsum(-1)[:, -1])  # order-free sums
    assert _single_rounding_differs(x) > 50


@pytest.mark.parametrize("H,offset", [(2048, 0), (2048, 1), (1000, 0)], ids=["chunks", "misaligned", "odd-width"])
def test_rmsnorm_rows_bit_exact(H, offset, dev):
    """lemoq_rmsnorm (16-byte chunk path and per-element path)."""
    print("case: rmsnorm rounding H=%d offset=%d" % (H, offset), flush=True)
    rows = 1024
    x, w = _rows(rows, H, H + offset)
    if H == 2048:
        assert _single_rounding_differs(x) > 0
    buf = torch.zeros(rows * H + 8, dtype=torch.float16, device=dev)
    xd = buf[offset:offset + rows * H].view(rows, H)
    xd.copy_(x.to(dev))
    wd = w.to(dev)
    y = torch.empty((rows, H), dtype=torch.float16, device=dev)
    _hip.call("lemoq_rmsnorm", _hip.ptr(xd), rows, H, _hip.ptr(wd), EPS, _hip.ptr(y), _hip.stream_of(dev))
    torch.cuda.synchronize()
    ref = ops.rms_norm(x, w, EPS)
    diff = int((_bits(y) != _bits(ref)).sum())
    assert diff == 0, "%d elements differ from the oracle" % diff


@pytest.mark.parametrize("K", [2048, 1024], ids=["block-norm", "wave-norm"])
def test_gemv_norm_prologue_bit_exact(K, dev):
    """lemoq_gemv_w8_fused's RMSNorm prologue (the block form for K >= 2048, the
    per-wave form below), observed through an identity weight matrix (code 1 on
    the diagonal, scale 1), so y is the normalised row itself."""
    print("case: gemv norm prologue rounding K=%d" % K, flush=True)
    rows = 256
    x, w = _rows(rows, K, K)
    codes = torch.zeros((K, K), dtype=torch.int8)
    codes[torch.arange(K), torch.arange(K)] = 1
    scale = torch.ones((K, K // 128), dtype=torch.float16)
    cd, sd, wd, xd = codes.to(dev), scale.to(dev), w.to(dev), x.to(dev)
    y = torch.empty((rows, K), dtype=torch.float16, device=dev)
    st = _hip.stream_of(dev)
    for r in range(rows):
        _hip.call("lemoq_gemv_w8_fused", _hip.ptr(xd[r]), None, 0, _hip.ptr(wd), EPS, None, _hip.ptr(cd),
                  _hip.ptr(sd), K, K, 128, None, _hip.ptr(y[r]), st)
    torch.cuda.synchronize()
    ref = ops.rms_norm(x, w, EPS)
    diff = int((_bits(y) != _bits(ref)).sum())
    assert diff == 0, "%d elements differ from the oracle" % diff


def test_router_norm_output_bit_exact(dev):
    """lemoq_router_logits_resid's xn (the post-attention RMSNorm feeding the
    router and the experts), with zero attention partials so h' = h."""
    print("case: router prologue norm rounding", flush=True)
    H, E, rows = 2048, 64, 128
    x, w = _rows(rows, H, 7)
    part = torch.zeros((1, H), dtype=torch.float32, device=dev)
    rw = torch.zeros((E, H), dtype=torch.float16, device=dev)
    wd = w.to(dev)
    xd = x.to(dev)
    xn = torch.empty((rows, H), dtype=torch.float16, device=dev)
    h_out = torch.empty(H, dtype=torch.float16, device=dev)
    lg = torch.empty(E, dtype=torch.float16, device=dev)
    st = _hip.stream_of(dev)
    for r in range(rows):
        _hip.call("lemoq_router_logits_resid", _hip.ptr(part), 1, _hip.ptr(xd[r]), _hip.ptr(wd), EPS, H,
                  _hip.ptr(rw), E, _hip.ptr(h_out), _hip.ptr(xn[r]), _hip.ptr(lg), st)
    torch.cuda.synchronize()
    ref = ops.rms_norm(x, w, EPS)
    diff = int((_bits(xn) != _bits(ref)).sum())
    assert diff == 0, "%d elements differ from the oracle" % diff


@pytest.mark.parametrize("K", [2048, 4096, 1024, 3072])
def test_gemv_q_norm_prologue_bit_exact(K, dev):
    """lemoq_gemv_q_rmsnorm's RMSNorm (the 4-bit decode step's input norm; the
    per-block form at K 2048 / 4096, the per-wave form at 1024 / 3072),
    observed through a 4-bit identity weight (code 1 on the diagonal, scale 1),
    all rows in one launch (M rows)."""
    print("case: 4-bit gemv norm prologue rounding K=%d" % K, flush=True)
    rows = 256
    x, w = _rows(rows, K, K + 5)
    packed = torch.zeros((K, K // 2), dtype=torch.uint8)
    r = torch.arange(K)
    packed[r, r // 2] = torch.where(r % 2 == 0, 1, 16).to(torch.uint8)  # code 1 in the row's own nibble
    scale = torch.ones((K, K // 128), dtype=torch.float16)
    pd, sd, wd, xd = packed.to(dev), scale.to(dev), w.to(dev), x.to(dev)
    y = torch.empty((rows, K), dtype=torch.float16, device=dev)
    _hip.call("lemoq_gemv_q_rmsnorm", _hip.ptr(xd), None, 0, rows, K, _hip.ptr(wd), EPS, None, _hip.ptr(pd), 2,
              _hip.ptr(sd), None, 0, K, K, 128, _hip.ptr(y), 1, _hip.stream_of(dev))
    torch.cuda.synchronize()
    ref = ops.rms_norm(x, w, EPS)
    diff = int((_bits(y) != _bits(ref)).sum())
    assert diff == 0, "%d elements differ from the oracle" % diff
