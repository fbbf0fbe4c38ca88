"""The fusion-switch mirror (``lemoq.kernels.fusion_switches``, the reference's
``src/lemoq/kernels/fusion_switches.py``): the same switch names, defaults and
environment overrides; every switch reports its requested state, and a switch
set to an arm this build does not have is refused, never ignored.  CPU only."""

from __future__ import annotations

import pytest

from lemoq.kernels import fusion_switches as fs


def test_names_defaults_and_overrides_match_the_reference():
    assert sorted(fs.ENV_VARS) == sorted(["fused_rope", "fused_route", "skip_mask_fill", "packed_qkv",
                                          "kv_direct_write", "lm_head_w8", "kv_int8"])
    assert fs.ENV_VARS["kv_int8"] == "LEMOQ_KV_INT8" and fs.ENV_VARS["lm_head_w8"] == "LEMOQ_LMHEAD_W8"
    assert fs.fusion_states({}) == {n: True for n in fs.ENV_VARS}
    assert fs.fusion_enabled("kv_int8", {"LEMOQ_KV_INT8": "0"}) is False
    assert fs.fusion_enabled("kv_int8", {"LEMOQ_KV_INT8": "1"}) is True
    assert fs.fusion_enabled("packed_qkv", {"LEMOQ_PACKED_QKV": "yes"}) is False  # only "1" is on
    assert fs.fusion_payload_fields({}) == fs.fusion_states({})
    with pytest.raises(KeyError):
        fs.fusion_enabled("fused_moe")


def test_only_built_arms_are_accepted():
    assert fs.require_built({})["kv_int8"] is True
    assert fs.require_built({"LEMOQ_KV_INT8": "0"})["kv_int8"] is False  # the fp16 cache is built
    with pytest.raises(NotImplementedError, match="packed_qkv"):
        fs.require_built({"LEMOQ_PACKED_QKV": "0"})
    with pytest.raises(NotImplementedError, match="LEMOQ_FUSED_ROPE, LEMOQ_LMHEAD_W8"):
        fs.require_built({"LEMOQ_LMHEAD_W8": "0", "LEMOQ_FUSED_ROPE": "0"})


def test_unavailable_reason_names_the_missing_device_here():
    import torch

    from lemoq.kernels import dequant_gemm, rmsnorm

    reason = rmsnorm.unavailable_reason()
    assert (reason is None) == rmsnorm.fused_available()
    if not torch.cuda.is_available():
        assert reason and dequant_gemm.unavailable_reason() == reason


def test_packed_qkv_switch_and_preconditions():
    from lemoq.kernels.packed_qkv import install_packed_qkv, packed_qkv_applicable, packed_qkv_enabled
    from torch import nn

    assert packed_qkv_enabled() is True
    assert packed_qkv_applicable("kernel", True) and not packed_qkv_applicable("sdpa", True)
    assert not packed_qkv_applicable("kernel", False)
    with pytest.raises(RuntimeError, match="no attention module"):
        install_packed_qkv(nn.Linear(4, 4))


def test_fuse_experts_stacks_gate_rows_first():
    """moe_static.fuse_experts (the reference's ``moe_static.py:106-122``): gate rows
    then up rows per expert, down as (E, H, F); host tensors stay host tensors."""
    import torch
    from torch import nn

    from lemoq.kernels.moe_static import FusedExperts, fuse_experts

    class _E(nn.Module):
        def __init__(self, i):
            super().__init__()
            self.gate_proj, self.up_proj, self.down_proj = nn.Linear(8, 4), nn.Linear(8, 4), nn.Linear(4, 8)
            for lin, off in ((self.gate_proj, 0), (self.up_proj, 100), (self.down_proj, 200)):
                nn.init.constant_(lin.weight, float(i + off))

    f = fuse_experts([_E(0), _E(1), _E(2)])
    assert isinstance(f, FusedExperts) and tuple(f.gate_up.shape) == (3, 8, 8) and tuple(f.down.shape) == (3, 8, 4)
    assert float(f.gate_up[2, 0, 0]) == 2.0 and float(f.gate_up[2, 4, 0]) == 102.0 and float(f.down[1, 0, 0]) == 201.0
    with pytest.raises(ValueError):
        fuse_experts([])
