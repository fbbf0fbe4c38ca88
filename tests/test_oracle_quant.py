"""Pins of the bit-exact CPU oracle functions (numpy, oracle/quant.py) — CPU only.

Each check is independent of the formula it pins: a second plain-C
restatement (oracle/c/quant_ref.c) written from the reference's contract,
hand-derived known-answer vectors (half-to-even ties, fp32-scale division),
and the invariants the reference's own tests assert
(tests/test_quant_oracle.py:107-163, tests/test_kv_int8.py:37-73,
tests/test_routing_fusion.py:24-52 of LeanMoE-Quant).
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from oracle import cref, ops
from oracle import quant as oq


@pytest.fixture(scope="module", autouse=True)
def _c_oracle():
    cref.build()


def _weights(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * 0.02


# ---------------------------------------------------------------------------
# RTN w8 (src/lemoq/quant/numpy_oracle.py:58-116, rtn.py:68-73)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("seed", [0, 1, 7, 2026])
@pytest.mark.parametrize("shape", [(64, 500), (3, 130), (1, 1), (16, 2048)])
@pytest.mark.parametrize("group", [128, 64, 32])
def test_rtn_numpy_equals_c_restatement(seed, shape, group):
    w = _weights(shape, seed)
    q = oq.rtn_quantize_w8(w, group)
    codes, s32, s16 = cref.rtn_w8(w, group)
    assert np.array_equal(q["codes_padded"], codes)
    assert np.array_equal(q["scale"], s32)
    assert np.array_equal(q["scale_f16"].view(np.uint16), s16.view(np.uint16))


@pytest.mark.parametrize(
    "w",
    [
        np.zeros((16, 40), dtype=np.float32),
        np.full((16, 40), np.finfo(np.float32).max, dtype=np.float32),
        np.full((16, 40), np.finfo(np.float32).tiny, dtype=np.float32),
    ],
    ids=["zeros", "finfo_max", "finfo_tiny"],
)
def test_rtn_edge_values_numpy_equals_c(w):
    for group in (32, 128):
        q = oq.rtn_quantize_w8(w, group)
        codes, s32, s16 = cref.rtn_w8(w, group)
        assert np.array_equal(q["codes_padded"], codes)
        assert np.array_equal(q["scale"], s32)
        assert np.array_equal(q["scale_f16"].view(np.uint16), s16.view(np.uint16))
    z = oq.rtn_quantize_w8(np.zeros((2, 40), np.float32), 32)
    assert (z["scale"] == 1.0).all() and (z["codes_padded"] == 0).all()


def test_rtn_known_answer_half_to_even():
    # amax 127 -> scale exactly 1.0: codes are the round-half-to-even of the values
    w = np.array([[127, -63.5, 0.5, 1.5, 2.5, -0.5, -1.5, 3.49, 3.5, -127, 100.5, 0, 64.5, -64.5, 126.5,
                   -126.5]], dtype=np.float32)
    q = oq.rtn_quantize_w8(w, 16)
    expect = [127, -64, 0, 2, 2, 0, -2, 3, 4, -127, 100, 0, 64, -64, 126, -126]
    assert q["codes_padded"].tolist() == [expect]
    assert q["scale"].tolist() == [[1.0]] and q["scale_f16"].tolist() == [[1.0]]


def test_rtn_divides_by_the_fp32_scale_not_the_fp16_one():
    # amax 1 -> s = 1/127 in fp32 (fp16(s) is 0.0078735...); 0.49999/s = 63.4987 -> 63,
    # while dividing by the fp16 scale would give 63.5026 -> 64.
    w = np.zeros((1, 16), np.float32)
    w[0, 0], w[0, 1] = 1.0, 0.49999
    q = oq.rtn_quantize_w8(w, 16)
    assert q["codes_padded"][0, :2].tolist() == [127, 63]
    assert q["scale"][0, 0] == np.float32(1.0) / np.float32(127.0)
    assert float(q["scale_f16"][0, 0]) == float(np.float16(np.float32(1.0) / np.float32(127.0)))


def test_rtn_invariants_and_padding():
    w = _weights((37, 500), 3)
    q = oq.rtn_quantize_w8(w, 128)
    c, s = q["codes_padded"].astype(np.int32), q["scale"]
    assert q["padded_in"] == 512 and c.shape == (37, 512)
    assert (c[:, 500:] == 0).all()                      # zero padding stays zero
    assert c.min() >= -127 and c.max() <= 127          # symmetric: -128 never produced
    g = np.abs(c.reshape(37, 4, 128)).max(axis=2)
    assert (g == 127).all()                              # each group's absmax hits 127
    rec = oq.rtn_dequant(q["codes_padded"], s, 128)[:, :500]
    bound = np.repeat(s, 128, axis=1)[:, :500] * 0.5 * (1 + 1e-5)
    assert (np.abs(rec - w) <= bound).all()


def test_rtn_fused_then_quantize_equals_per_expert():
    """Quantising the stacked experts equals quantising each expert (groups are
    row-local), the invariant of tests/test_moe_grouped_quant.py:76-114."""
    e, rows, cols = 4, 16, 256
    w = _weights((e * rows, cols), 11)
    whole = oq.rtn_quantize_w8(w, 128)
    for i in range(e):
        part = oq.rtn_quantize_w8(w[i * rows:(i + 1) * rows], 128)
        assert np.array_equal(whole["codes_padded"][i * rows:(i + 1) * rows], part["codes_padded"])
        assert np.array_equal(whole["scale"][i * rows:(i + 1) * rows], part["scale"])


# ---------------------------------------------------------------------------
# KV-INT8 per-token quantisation (src/lemoq/kernels/kv_int8.py:30-41, :196-216)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("seed", range(4))
def test_kv_numpy_equals_c_restatement(seed):
    x = (np.random.default_rng(seed).standard_normal((16, 37, 128)) * 3).astype(np.float16)
    x[0, 0] = 0  # a zero row
    c1, s1 = oq.kv_quantize_rows(x)
    c2, s2 = cref.kv_quant_rows(x)
    assert np.array_equal(c1, c2)
    assert np.array_equal(s1.view(np.uint16), s2.view(np.uint16))


def test_kv_known_answer():
    x = np.array([[2.0, 1.0, 0.5, -1.0, -2.0, 0.25, 0.0078125, -0.0078125]], dtype=np.float16)
    c, s = oq.kv_quantize_rows(x)
    # s = 2/127; 1/s = 63.5 exactly in fp32 -> 64 (half to even); 0.5/s = 31.75 -> 32
    assert c.tolist() == [[127, 64, 32, -64, -127, 16, 0, 0]]
    assert s.view(np.uint16).tolist() == [np.float16(np.float32(2) / np.float32(127)).view(np.uint16)]


def test_kv_scale_formula_zero_row_range_and_lead():
    x = (np.random.default_rng(5).standard_normal((16, 128))).astype(np.float16)
    c, s = oq.kv_quantize_rows(x)
    expect = (np.abs(x.astype(np.float32)).max(axis=-1) / np.float32(127)).astype(np.float16)
    assert np.array_equal(s.view(np.uint16), expect.view(np.uint16))
    assert c.min() >= -127 and c.max() <= 127
    lead = np.take_along_axis(c.astype(np.int32), np.abs(x.astype(np.float32)).argmax(-1)[:, None], -1)
    assert (np.abs(lead) == 127).all()
    zc, zs = oq.kv_quantize_rows(np.zeros((3, 128), np.float16))
    assert (zs == 1.0).all() and (zc == 0).all()


@pytest.mark.parametrize("seed", range(4))
def test_kv_roundtrip_bound(seed):
    x = (np.random.default_rng(seed).standard_normal((16, 128))).astype(np.float16)
    c, s = oq.kv_quantize_rows(x)
    rec = c.astype(np.float32) * s.astype(np.float32)[:, None]
    # |err| <= s/2 + fp16 rounding of s (127 * 2^-11 * s) < 0.6 s  (tests/test_kv_int8.py:64-73)
    assert (np.abs(rec - x.astype(np.float32)) <= 0.6 * s.astype(np.float32)[:, None]).all()


# ---------------------------------------------------------------------------
# Routing order (src/lemoq/kernels/_routing_triton.py:11-14, 55-80)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("e,k", [(64, 8), (8, 2), (60, 4)])
def test_route_torch_oracle_equals_numpy_oracle(norm, e, k):
    z = torch.randn((32, e), generator=torch.Generator().manual_seed(e * k)) * 2
    wn, idn = oq.route_order(z.numpy(), k, norm)
    logits, wt, it = ops.route(z, torch.eye(e), k, norm)  # F.linear(z, I) == z
    assert np.array_equal(it.numpy(), idn)
    assert np.allclose(wt.numpy(), wn, rtol=1e-6, atol=1e-7)


def test_route_brute_force_ties_lowest_index():
    # every assignment of 6 experts to values {0, 1, 2}: the top-3 must be the
    # order (value desc, index asc), found here by exhaustive comparison
    for vals in itertools.product([0.0, 1.0, 2.0], repeat=6):
        z = np.array([vals], dtype=np.float32)
        _, idx = oq.route_order(z, 3, False)
        best = sorted(range(6), key=lambda i: (-vals[i], i))[:3]
        assert idx[0].tolist() == best, vals


def test_route_renorm_sums_to_one_and_weights_are_softmax_values():
    z = np.random.default_rng(9).standard_normal((8, 64)).astype(np.float32)
    w, idx = oq.route_order(z, 8, True)
    assert np.allclose(w.sum(-1), 1.0, atol=1e-6)
    w0, idx0 = oq.route_order(z, 8, False)
    assert np.array_equal(idx, idx0)
    p = np.exp(z.astype(np.float64) - z.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    assert np.allclose(w0, np.take_along_axis(p, idx0, -1), rtol=1e-5)
