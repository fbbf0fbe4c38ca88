"""The stable quantisation entry points (``lemoq.quant``, the reference's
``src/lemoq/quant/api.py``) on the CPU: the ladder's shape and the argument
refusals, which happen before anything touches a device."""

from __future__ import annotations

import pytest
import torch

import lemoq.quant as lq


def test_remediation_ladder_order_and_what_is_built():
    steps = [s["step"] for s in lq.REMEDIATION_LADDER]
    assert steps == ["1_rtn", "2_gptq", "3_awq", "4_mixed_bits", "5_selective"]
    assert all({"step", "method", "needs_calibration", "built_here"} <= set(s) for s in lq.REMEDIATION_LADDER)
    assert [s["needs_calibration"] for s in lq.REMEDIATION_LADDER] == ["no", "yes", "yes", "yes", "no"]


def test_quantize_linear_refusals_come_first():
    w = torch.zeros((4, 128))
    with pytest.raises(NotImplementedError, match="awq"):
        lq.quantize_linear(w, scheme="awq")
    with pytest.raises(NotImplementedError, match="calibration"):
        lq.quantize_linear(w, scheme="gptq", calibration=torch.zeros(2, 128))
    with pytest.raises(ValueError, match="calibration"):
        lq.quantize_linear(w, scheme="rtn", calibration=torch.zeros(2, 128))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        lq.quantize_linear(w, bits=8)  # the quantiser runs on the device only
    q = lq.QuantizedLinear(codes=None, scale=None, zero=None, bits=8, group_size=128, symmetric=True,
                           scheme="rtn", shape=(6, 300))
    assert q.n_params == 1800
