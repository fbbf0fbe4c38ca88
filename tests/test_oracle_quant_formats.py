"""Pins the CPU oracle of the weight formats beyond 8-bit symmetric
(``oracle.quant``: ``rtn_quantize``, ``pack_4bit`` / ``unpack_4bit``,
``dequant_tile``, ``mxfp4_quantize`` / ``mxfp4_dequantize``).

Checks, each chosen so that a plausible slip fails it:

1. ``rtn_quantize`` equals an independent plain-C restatement
   (``oracle/c/quant_ref.c:oracle_rtn``) bit for bit over the reference's own
   case grid (``tests/test_quant_oracle.py:104-146``: bits 4/8, several groups,
   non-divisible widths, seeds, all-zero / largest / smallest-normal weights),
   symmetric and asymmetric; hand-computed codes on exactly representable
   inputs; the round-trip error bounds (symmetric <= s/2, asymmetric <= s); the
   asymmetric range over the real columns only (the padding of the last group
   left out, ``src/lemoq/quant/rtn.py:62-75``).
2. ``pack_4bit`` / ``unpack_4bit``: known bytes (low nibble first) and round
   trips, signed and unsigned (``src/lemoq/quant/pack.py:21-63``).
3. ``dequant_tile`` equals the fp64 product rounded once to fp32.
4. ``mxfp4_*``: the reference's known answers (``tests/test_mxfp4.py``: the
   E2M1 table, the E8M0 bias, the 0..6 ladder, saturation at 7.9, the 0.1
   block, signs, the all-zero block, the 2-scale error bound, padding to 32),
   every E8M0 byte dequantising to exactly 2^(X - 127) (numpy's float32 exp2
   is an ulp off at 127, torch's, which the reference uses, is exact),
   a brute-force nearest-code check, and the C restatement
   (``oracle_mxfp4``, log2 in long double) bit for bit, including amax one to
   five ulps below powers of two, where torch's fp32 log2 rounds up to the
   integer (the floor then sees k, not k - 1).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import cref
from oracle import quant as oq

CASES = [(4, 128, True), (4, 32, True), (8, 128, True), (8, 64, True), (4, 128, False), (8, 128, False),
         (4, 64, False), (8, 32, False)]


def _weights(shape=(64, 256), seed=0):
    return (np.random.default_rng(seed).standard_normal(shape) * 0.05).astype(np.float32)


@pytest.mark.parametrize("bits,group,sym", CASES)
@pytest.mark.parametrize("shape,seed", [((64, 256), 0), ((64, 500), 1), ((3, 130), 7), ((1, 1), 2026),
                                        ((16, 40), 3)])
def test_rtn_matches_the_c_restatement(bits, group, sym, shape, seed):
    w = _weights(shape, seed)
    q = oq.rtn_quantize(w, bits, group, sym)
    c, s, z = cref.rtn(w, group, bits, sym)
    assert np.array_equal(q["codes_padded"], c)
    assert np.array_equal(q["scale"], s) and np.array_equal(q["zero"], z)


@pytest.mark.parametrize("fill", [0.0, float(np.finfo(np.float32).max), float(np.finfo(np.float32).tiny)],
                         ids=["zeros", "finfo_max", "finfo_tiny"])
@pytest.mark.parametrize("bits,group,sym", [(4, 128, True), (8, 32, True), (4, 128, False), (8, 32, False)])
def test_rtn_edge_values_match_the_c_restatement(fill, bits, group, sym):
    w = np.full((16, 40), fill, dtype=np.float32)
    q = oq.rtn_quantize(w, bits, group, sym)
    c, s, z = cref.rtn(w, group, bits, sym)
    assert np.array_equal(q["codes_padded"], c)
    assert np.array_equal(q["scale"], s) and np.array_equal(q["zero"], z)


def test_rtn_known_codes_on_exact_inputs():
    # symmetric 4-bit: absmax 2.625 -> s = 0.375 exactly; w / s = 2, -4, 1, 7
    q = oq.rtn_quantize(np.array([[0.75, -1.5, 0.375, 2.625]], np.float32), 4, 4, True)
    assert q["scale"][0, 0] == np.float32(0.375)
    assert q["codes_padded"].tolist() == [[2, -4, 1, 7]]
    # asymmetric 4-bit: range 3.75 -> s = 0.25, zero = round(1 / 0.25) = 4
    q = oq.rtn_quantize(np.array([[-1.0, -0.5, 0.0, 2.75]], np.float32), 4, 4, False)
    assert q["scale"][0, 0] == np.float32(0.25) and q["zero"][0, 0] == 4.0
    assert q["codes_padded"].tolist() == [[0, 2, 4, 15]]
    # 8-bit symmetric: the negative end reaches -128 only by clamping, round half to even
    q = oq.rtn_quantize(np.array([[1.0, -1.0, 0.5 / 127 * 1.0, 2.5 / 127]], np.float32), 8, 4, True)
    assert q["codes_padded"].tolist() == [[127, -127, 0, 2]]


@pytest.mark.parametrize("bits,group,sym", CASES)
def test_rtn_round_trip_error_bounds(bits, group, sym):
    w = _weights((32, 300), 5)
    q = oq.rtn_quantize(w, bits, group, sym)
    deq = oq.dequant_tile(q["codes_padded"], q["scale"], q["zero"], group, sym, in_features=300)
    s = np.repeat(q["scale"], group, axis=1)[:, :300]
    err = np.abs(deq.astype(np.float64) - w)
    assert np.all(err <= (0.5 if sym else 1.0) * s * (1 + 1e-6) + 1e-12)
    qmax = 2 ** (bits - 1) - 1 if sym else 2 ** bits - 1
    lo = -(qmax + 1) if sym else 0
    assert q["codes_padded"].min() >= lo and q["codes_padded"].max() <= qmax
    assert np.array_equal(q["zero"], np.round(q["zero"]))


def test_rtn_asymmetric_range_leaves_the_padding_out():
    """All-positive rows of width 130 in groups of 128: the last group's two real
    columns set its range; counting the zero padding would make min 0."""
    w = (np.abs(_weights((3, 130), 9)) + 1.0).astype(np.float32)
    q = oq.rtn_quantize(w, 4, 128, False)
    tail = w[:, 128:]
    want = np.where(tail.max(1) > tail.min(1), (tail.max(1) - tail.min(1)) / np.float32(15), 1.0)
    assert np.array_equal(q["scale"][:, 1], want.astype(np.float32))
    padded_min = np.minimum(tail.min(1), 0.0)
    assert not np.array_equal(q["scale"][:, 1], ((tail.max(1) - padded_min) / np.float32(15)).astype(np.float32))


def test_pack_known_bytes_and_round_trips():
    assert oq.pack_4bit(np.array([[1, -1, 7, -8]])).tolist() == [[0xF1, 0x87]]
    rng = np.random.default_rng(4)
    c = rng.integers(-8, 8, (5, 64))
    assert np.array_equal(oq.unpack_4bit(oq.pack_4bit(c), signed=True), c)
    u = rng.integers(0, 16, (5, 64))
    assert np.array_equal(oq.unpack_4bit(oq.pack_4bit(u), signed=False), u)
    assert oq.unpack_4bit(np.array([[0xF1]], np.uint8), signed=True).tolist() == [[1, -1]]
    assert oq.unpack_4bit(np.array([[0xF1]], np.uint8), signed=False).tolist() == [[1, 15]]


@pytest.mark.parametrize("sym", [True, False])
def test_dequant_tile_is_one_rounding_of_the_exact_product(sym):
    rng = np.random.default_rng(8)
    codes = rng.integers(0 if not sym else -8, 16 if not sym else 8, (6, 128))
    scale = (rng.random((6, 4)) * 0.1 + 1e-3).astype(np.float16)
    zero = rng.integers(0, 16, (6, 4)).astype(np.float16)
    got = oq.dequant_tile(codes, scale, zero, 32, sym)
    c64 = codes.astype(np.float64).reshape(6, 4, 32)
    s64 = scale.astype(np.float64)[:, :, None]
    z64 = zero.astype(np.float64)[:, :, None]
    want = ((c64 if sym else c64 - z64) * s64).reshape(6, 128).astype(np.float32)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------------------
# MXFP4
# ---------------------------------------------------------------------------
def _mx_roundtrip(w):
    q = oq.mxfp4_quantize(w)
    return q, oq.mxfp4_dequantize(q["codes_packed"], q["scales"], q["orig_in"])


def test_e2m1_table_and_e8m0_bias():
    want = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    codes = np.array([list(range(16)) * 2], dtype=np.uint8)
    for byte, scale in ((127, 1.0), (128, 2.0), (126, 0.5), (0, 2.0 ** -127)):
        got = oq.mxfp4_dequantize(oq.pack_4bit(codes), np.array([[byte]], np.uint8), 32)
        assert got[0, :16].tolist() == [v * scale for v in want]
        assert np.signbit(got[0, 8])  # code 8 is -0


def test_e8m0_scale_is_the_exact_power_of_two_for_every_byte():
    """Every scale byte 0..254 at code 2 (1.0) dequantises to exactly 2^(X-127),
    the largest (2^127) included; byte 255 is 2^128 = inf in fp32."""
    codes = np.full((256, 32), 2, np.uint8)
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    got = oq.mxfp4_dequantize(oq.pack_4bit(codes), scales, 32)[:, 0]
    for X in range(255):
        assert got[X] == np.float32(2.0 ** (X - 127)), X
    assert np.isinf(got[255])


def test_ladder_block_round_trips_exactly():
    w = np.array([list(oq.E2M1_MAG) + [0.0] * 24], np.float32)
    q, dq = _mx_roundtrip(w)
    assert q["scales"][0, 0] == 127 and np.array_equal(dq, w)


def test_saturation_small_block_signs_and_zero_block():
    q, dq = _mx_roundtrip(np.array([[7.9] + [0.0] * 31], np.float32))  # floor(log2 7.9) - 2 = 0
    assert q["scales"][0, 0] == 127 and dq[0, 0] == 6.0 and abs(7.9 - dq[0, 0]) < 2.0
    q, dq = _mx_roundtrip(np.array([[0.1] + [0.0] * 31], np.float32))  # floor(log2 0.1) = -4 -> X = -6
    assert q["scales"][0, 0] == 121 and dq[0, 0] == np.float32(6.0 * 2.0 ** -6)
    q, dq = _mx_roundtrip(np.array([[-3.0, 3.0] + [0.0] * 30], np.float32))  # X = -1, 3 / 0.5 = 6
    assert dq[0, 0] == -3.0 and dq[0, 1] == 3.0
    q, dq = _mx_roundtrip(np.zeros((1, 32), np.float32))
    assert q["scales"][0, 0] == 0 and not dq.any()


def test_random_error_bound_and_padding():
    w = (np.random.default_rng(0).standard_normal((8, 128)) * 0.3).astype(np.float32)
    q, dq = _mx_roundtrip(w)
    s = np.repeat(np.exp2(q["scales"].astype(np.float64) - 127), 32, axis=1)
    assert np.all(np.abs(dq - w) <= 2.0 * s + 1e-12)
    w = (np.random.default_rng(3).standard_normal((4, 50)) * 0.2).astype(np.float32)
    q, dq = _mx_roundtrip(w)
    assert q["padded_in"] == 64 and q["codes_packed"].shape == (4, 32) and q["scales"].shape == (4, 2)
    assert dq.shape == (4, 50)


def test_codes_are_the_first_nearest_magnitude():
    """Brute force: |v| clamped to 6 against every magnitude, the first of the
    closest wins (ties go to the smaller magnitude); the sign bit is v < 0."""
    w = (np.random.default_rng(11).standard_normal((16, 96)) * 0.7).astype(np.float32)
    w[0, :8] = [0.25, -0.25, 1.25, 2.5, -3.5, 5.0, 0.75, -1.75]  # exact ties in block 0 (amax 5 -> X = 0)
    q = oq.mxfp4_quantize(w)
    X = q["scales"].astype(np.int64) - 127
    v = w / np.repeat(np.exp2(X.astype(np.float64)), 32, axis=1)
    mags = np.asarray(oq.E2M1_MAG)
    for (r, k), val in np.ndenumerate(v):
        m = min(abs(val), 6.0)
        d = [abs(m - x) for x in mags]
        best = min(range(8), key=lambda i: (d[i], i))
        assert q["codes"][r, k] == ((8 if val < 0 else 0) | best), (r, k, val)
    assert q["codes"][0, :8].tolist() == [0, 8, 2, 4, 8 | 5, 6, 1, 8 | 3]


def test_mxfp4_matches_the_c_restatement_at_power_of_two_edges():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((64, 256)) * 0.3).astype(np.float32)
    rows = []
    for k in range(-20, 21):
        a = np.float32(2.0 ** k)
        for _ in range(5):  # amax 1..5 ulps below 2^k, and 2^k itself
            a = np.nextafter(a, np.float32(0))
            blk = np.zeros(32, np.float32)
            blk[3] = a
            blk[7] = -a * np.float32(0.3)
            rows.append(blk)
        blk = np.zeros(32, np.float32)
        blk[0] = np.float32(2.0 ** k)
        rows.append(blk)
    w_edge = np.stack(rows)
    for ww in (w, w_edge, w * np.float32(1e-30), np.zeros((2, 70), np.float32)):
        q = oq.mxfp4_quantize(ww)
        c, s = cref.mxfp4(ww)
        assert np.array_equal(q["codes"], c) and np.array_equal(q["scales"], s)
