"""CPU tests of the host-side helpers of the operator surface: launch geometry,
split-count default, the length-change verdict, the frozen gates, the KV-INT8
row guard and the quantised-expert container.  Mirrors the reference's own
host tests (tests/test_attn_decode.py:155-233, tests/test_moe_grouped_quant.py)
with hand-computed values; nothing here launches a kernel."""

from __future__ import annotations

import math

import pytest
import torch

from lemoq.kernels import attn_decode as ad
from lemoq.kernels import kv_int8
from lemoq.kernels.moe_grouped_quant import QuantFusedExperts


def test_launch_plan_hand_computed():
    plan = ad.launch_plan(heads=16, head_dim=128, num_splits=10, block_n=128)
    assert plan["kernel_count"] == 2
    assert plan["split"]["grid"] == (10, 16)
    assert plan["split"]["m_shape"] == (16, 10)
    assert plan["split"]["l_shape"] == (16, 10)
    assert plan["split"]["acc_shape"] == (16, 10, 128)
    assert plan["split"]["dtype"] == "float32"
    assert plan["combine"]["grid"] == (16,)
    assert plan["combine"]["out_shape"] == (1, 16, 1, 128)
    assert (plan["heads"], plan["head_dim"], plan["num_splits"]) == (16, 128, 10)


@pytest.mark.parametrize("kw", [
    dict(heads=16, head_dim=128, num_splits=10, block_n=100),   # tile not a power of two
    dict(heads=16, head_dim=100, num_splits=10),                # head_dim not a power of two
    dict(heads=16, head_dim=128, num_splits=0),
    dict(heads=0, head_dim=128, num_splits=4),
    dict(heads=16, head_dim=128, num_splits=4, block_d=64),     # block_d below head_dim
])
def test_launch_plan_rejects_illegal_shapes(kw):
    with pytest.raises(ValueError):
        ad.launch_plan(**kw)


def test_resolve_num_splits_defaults_and_overrides(monkeypatch):
    assert ad.resolve_num_splits(7, heads=16) == 7
    with pytest.raises(ValueError):
        ad.resolve_num_splits(0, heads=16)
    # no device visible: 1
    monkeypatch.setattr(ad, "_device_cu_count", lambda device: 0)
    assert ad.resolve_num_splits(None, heads=16) == 1
    # MI355X: 256 CUs / 16 heads; a count that does not divide rounds up
    monkeypatch.setattr(ad, "_device_cu_count", lambda device: 256)
    assert ad.resolve_num_splits(None, heads=16) == 16
    monkeypatch.setattr(ad, "_device_cu_count", lambda device: 170)
    assert ad.resolve_num_splits(None, heads=16) == 11
    assert ad.resolve_num_splits(None, heads=0) == 170


def test_merged_config_overlays_without_touching_defaults():
    before = dict(ad.ATTN_CONFIGS)
    cfg = ad.merged_config({"num_splits": 4, "split": {"BLOCK_N": 64}})
    assert cfg["num_splits"] == 4 and cfg["split"] == {"BLOCK_N": 64}
    assert ad.ATTN_CONFIGS == before and ad.merged_config() == before
    # a dict override updates a dict default one level deep
    ad.ATTN_CONFIGS["tile"] = {"a": 1, "b": 2}
    try:
        assert ad.merged_config({"tile": {"b": 3}})["tile"] == {"a": 1, "b": 3}
        assert ad.ATTN_CONFIGS["tile"] == {"a": 1, "b": 2}
    finally:
        del ad.ATTN_CONFIGS["tile"]


def test_gates_are_frozen():
    assert ad.PARITY_GATE["tol_atol"] == 1e-3
    assert ad.PARITY_GATE["tol_rtol"] == 1e-3
    assert ad.PARITY_GATE["tol_slack"] == 1.5
    assert ad.LENGTH_CHANGE_GATE["correct_err_max"] == 1e-2
    assert ad.LENGTH_CHANGE_GATE["discriminant_min"] == 1.0
    assert ad.ATTN_CONFIGS["num_splits"] is None
    assert abs(ad.LOG2E - 1.0 / math.log(2.0)) < 1e-15


def test_length_change_verdicts():
    ok = ad.judge_length_change(correct_err=1e-4, stale_err=5.0)
    assert ok["verdict"] == "PASS" and ok["discriminating"] is True
    # the stale answer reported as the answer must fail
    assert ad.judge_length_change(correct_err=5.0, stale_err=5.0)["verdict"] == "FAIL"
    # no discriminating power: inconclusive, never PASS
    nd = ad.judge_length_change(correct_err=1e-6, stale_err=1e-6)
    assert nd["verdict"] == "INCONCLUSIVE" and nd["discriminating"] is False
    # thresholds: correct_err must be strictly below, stale_err at least the discriminant
    assert ad.judge_length_change(correct_err=1e-2, stale_err=1.0)["verdict"] == "FAIL"
    edge = ad.judge_length_change(correct_err=0.0, stale_err=1.0)
    assert edge["verdict"] == "PASS" and edge["gate"] == ad.LENGTH_CHANGE_GATE
    custom = ad.judge_length_change(correct_err=0.5, stale_err=3.0,
                                    gate={"correct_err_max": 1.0, "discriminant_min": 2.0})
    assert custom["verdict"] == "PASS"


def test_kv_row_guard_on_cpu_tensors():
    k = torch.zeros(1, 16, 1, 128, dtype=torch.float16)
    # CPU rows never take the device write path, even at the right shape
    assert kv_int8.kv_int8_rows_applicable(k, k.clone()) is False
    assert kv_int8._row_guard_failure(k, k) == "k/v are not on the GPU"
    assert kv_int8._row_guard_failure(k, None) == "k/v are not tensors"
    with pytest.raises(RuntimeError, match="row guard failed"):
        kv_int8.kv_int8_write(k, k)


def _experts(e=3, f=32, h=64, g=32):
    gen = torch.Generator().manual_seed(0)
    return QuantFusedExperts(
        packed_gate_up=torch.randint(-127, 128, (e, 2 * f, h), dtype=torch.int8, generator=gen),
        scale_gate_up=torch.rand(e, 2 * f, h // g, generator=gen).half(),
        packed_down=torch.randint(-127, 128, (e, h, f), dtype=torch.int8, generator=gen),
        scale_down=torch.rand(e, h, f // g, generator=gen).half(),
        bits=8, group_size=g)


def test_quant_fused_experts_container():
    q = _experts()
    assert (q.num_experts, q.ffn, q.hidden) == (3, 32, 64)
    # codes 1 byte each, scales 2 bytes per group of 32
    assert q.nbytes() == 3 * 64 * 64 + 2 * 3 * 64 * 2 + 3 * 64 * 32 + 2 * 3 * 64 * 1
    assert q.to() is q
    moved = q.to("cpu")
    assert moved is not q and moved.bits == 8 and moved.group_size == 32
    assert torch.equal(moved.packed_down, q.packed_down) and moved.scale_gate_up.dtype == torch.float16
    # a dtype change would undo the quantisation: refused, positional or keyword
    with pytest.raises(ValueError):
        q.to(torch.float32)
    with pytest.raises(ValueError):
        q.to("cpu", dtype=torch.float16)
