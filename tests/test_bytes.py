"""Byte model of the decode step (CPU).

Anchors are the reference's own (tests/test_bytes.py:39-79 of LeanMoE-Quant,
EXP-p4c-01-in-graph-attention.md:152) and the per-call figures of the
hot-path kernels; the KV-INT8 term counts int8 codes + fp16 scales.
"""

from __future__ import annotations

import pytest

from lemoq.bytes import WeightBits, attainment, kv_read_bytes, step_bytes, weight_budget
from lemoq.model.olmoe import OLMOE_1B_7B

FP16 = WeightBits(attention=16, experts=16, lm_head=16)


def test_fp16_W_anchor_and_shares():
    w = weight_budget(OLMOE_1B_7B, FP16)
    assert w["total_bytes"] == 2_357_723_136
    by = {it["name"]: it for it in w["items"]}
    assert by["experts(top-k)"]["share_pct"] == pytest.approx(68.3, abs=0.1)
    assert by["attention"]["share_pct"] == pytest.approx(22.8, abs=0.1)
    assert by["lm_head"]["share_pct"] == pytest.approx(8.7, abs=0.1)
    assert by["router"]["share_pct"] == pytest.approx(0.2, abs=0.1)
    assert by["embedding_row"]["counted_in_total"] is False and by["embedding_row"]["bytes"] == 4096


def test_w8_with_fp16_lm_head_matches_reference_total():
    w = weight_budget(OLMOE_1B_7B, WeightBits(attention=8, experts=8, lm_head=16))
    assert w["total_bytes"] == 1_300_758_528


def test_canonical_w8_cell_and_per_call_bytes():
    w = weight_budget(OLMOE_1B_7B)
    assert w["total_bytes"] == 1_199_345_664
    by = {it["name"]: it["bytes"] for it in w["items"]}
    # per call: qkv 12,779,520 + o_proj 4,259,840 per layer; 8 experts 51,118,080 per layer
    assert by["attention"] == 16 * (12_779_520 + 4_259_840)
    assert by["experts(top-k)"] == 16 * 51_118_080
    assert by["lm_head"] == 104_632_320
    assert w["streamed_bytes"] - w["total_bytes"] == 270_336
    # the model's own accounting agrees
    assert OLMOE_1B_7B.weight_bytes_per_token() == w["streamed_bytes"]


def test_kv_anchors_fp16_and_int8():
    assert kv_read_bytes(OLMOE_1B_7B, 1024, kv="fp16") == 134_217_728
    assert kv_read_bytes(OLMOE_1B_7B, 4096, kv="fp16") == 536_870_912
    # KV-INT8: 4160 B per token and layer (16 heads x (128 + 2) x K,V)
    assert kv_read_bytes(OLMOE_1B_7B, 1, kv="int8") == 16 * 4160
    assert kv_read_bytes(OLMOE_1B_7B, 4096, kv="int8") // 16 == 17_039_360
    assert kv_read_bytes(OLMOE_1B_7B, 2048, kv="fp16", batch=4) == 4 * 2 * 134_217_728


def test_step_bytes_and_attainment():
    b1 = step_bytes(OLMOE_1B_7B, 1025)
    assert b1 == 1_199_345_664 + 270_336 + 66_560 * 1025
    assert abs(b1 / 1e9 - 1.268) < 0.001
    assert attainment(1e9, 1e-3, 2e12) == pytest.approx(0.5)
    with pytest.raises(ValueError):
        attainment(1.0, 0.0, 1.0)
    with pytest.raises(ValueError):
        kv_read_bytes(OLMOE_1B_7B, 10, kv="fp8")


def test_step_split_rule():
    """One split per 64 cache slots, at least 2, and heads * splits within one
    block per compute unit (a second round of blocks costs more than it saves)."""
    from lemoq.model.olmoe import step_num_splits

    assert step_num_splits(1061, 16, 256) == 16 and step_num_splits(4133, 16, 256) == 16
    assert step_num_splits(20, 2, 256) == 2 and step_num_splits(300, 2, 256) == 5
    assert step_num_splits(100000, 4, 256) == 64 and step_num_splits(5000, 16, 128) == 8
    for S in (1, 63, 64, 65, 1000, 5000):
        for heads in (1, 2, 16, 64, 300):
            ns = step_num_splits(S, heads, 256)
            assert ns >= 1 and (heads * ns <= 256 or ns == 1)


def test_w4a16_cell_bytes():
    """The w4a16 cell (attention + experts at 4 bits, router and lm_head fp16):
    the reference's anchors (tests/test_bytes.py:88-105 of LeanMoE-Quant) -- the
    fp16 lm_head streams 103,022,592 x 2 bytes and the whole [W] shrinks by less
    than 4x against fp16 -- and the per-call figures the 4-bit kernels move."""
    bits = WeightBits(attention=4, experts=4, lm_head=16)
    w = weight_budget(OLMOE_1B_7B, bits)
    by = {it["name"]: it["bytes"] for it in w["items"]}
    assert by["lm_head"] == 103_022_592 * 2
    assert 2.5 < weight_budget(OLMOE_1B_7B, FP16)["total_bytes"] / w["total_bytes"] < 4.0
    # per layer: q|k|v 6144 x 1024 codes + 6144 x 16 scales, o_proj 2048 x 1024 + 2048 x 16,
    # 8 experts x (2048 x 1024 + 2048 x 16 gate/up, 2048 x 512 + 2048 x 8 down)
    assert by["attention"] == 16 * ((6144 * 1024 + 6144 * 32) + (2048 * 1024 + 2048 * 32))
    assert by["experts(top-k)"] == 16 * 8 * ((2048 * 1024 + 2048 * 32) + (2048 * 512 + 2048 * 16))
    assert w["total_bytes"] == by["attention"] + by["experts(top-k)"] + by["lm_head"] + by["router"]
    with pytest.raises(ValueError):
        weight_budget(OLMOE_1B_7B, WeightBits(attention=3))
