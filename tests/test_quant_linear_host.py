"""Host logic of the QuantLinear surface around the decode path (CPU only):
the reference's name classification (``src/lemoq/quant/linear.py:214-243``),
``SchemeSpec.to_dict``, ``quantize_model``'s skip rules and report, the
dispatch counters and the fallback reasons, and that a CPU input fails loudly
(this build has no CPU arm) without counting a call."""

from __future__ import annotations

import pytest
import torch
from torch import nn

from lemoq.quant.linear import (
    QuantLinear,
    SchemeSpec,
    classify_linear,
    dequant_activity,
    quantize_model,
    realized_bytes,
    reset_dequant_counters,
    set_dequant_mode,
    supported_dequant_modes,
)
from lemoq.quant.linear import _layer_index


def test_classify_linear_follows_the_reference_names():
    assert classify_linear("lm_head") == "lm_head"
    assert classify_linear("model.layers.3.self_attn.q_proj") == "attention"
    assert classify_linear("model.layers.0.self_attn.o_proj") == "attention"
    assert classify_linear("model.layers.0.mlp.experts.17.gate_proj") == "experts"
    assert classify_linear("model.layers.5.mlp.gate") == "router"
    assert classify_linear("model.layers.5.mlp.gate_proj") is None  # a dense MLP is no target
    assert classify_linear("model.layers.2.mlp.shared_expert.up_proj") == "shared"
    assert classify_linear("model.embed_tokens") is None
    assert classify_linear("encoder.lm_head") is None  # only the top-level lm_head
    assert (_layer_index("model.layers.12.mlp.gate"), _layer_index("lm_head")) == (12, None)


def test_spec_to_dict_carries_the_reference_keys():
    d = SchemeSpec.from_flags("w8a8", 64).to_dict()
    assert set(d) == {"scheme", "weight_bits", "act_bits", "group_size", "targets", "keep_lm_head_fp16",
                      "symmetric", "rtn_scheme", "dequant", "activation_quantization"}
    assert (d["weight_bits"], d["act_bits"], d["group_size"], d["rtn_scheme"]) == (8, 8, 64, "rtn")
    assert d["activation_quantization"] and SchemeSpec.from_flags("w8a16", 64).to_dict()["activation_quantization"] is None
    assert SchemeSpec.from_flags("mxfp4", 128).to_dict()["group_size"] == 32


class _Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn = nn.Module()
        self.self_attn.q_proj = nn.Linear(8, 8)
        self.mlp = nn.Module()
        self.mlp.gate = nn.Linear(8, 4, bias=False)


def _model():
    m = nn.Module()
    m.model = nn.Module()
    m.model.layers = nn.ModuleList([_Layer(), _Layer()])
    m.lm_head = nn.Linear(8, 16, bias=False)
    return m


def test_quantize_model_skips_with_reasons_and_a_disabled_spec_changes_nothing():
    m = _model()
    _, rep = quantize_model(m, SchemeSpec.from_flags("fp16", 128))
    assert rep.replaced == {} and rep.skipped == [] and isinstance(m.lm_head, nn.Linear)
    # nothing here is quantised (no target matches, or filtered out): no device needed
    spec = SchemeSpec.from_flags("w8a16", 128, targets=("experts",))
    _, rep = quantize_model(m, spec)
    assert rep.replaced == {}
    assert "model.layers.0.self_attn.q_proj (target=attention not in spec.targets)" in rep.skipped
    assert "lm_head (target=lm_head not in spec.targets)" in rep.skipped
    spec = SchemeSpec.from_flags("w8a16", 128, targets=("lm_head", "router"), keep_lm_head_fp16=True)
    _, rep = quantize_model(m, spec, layers=[7])
    assert "lm_head (keep_lm_head_fp16=True)" in rep.skipped
    assert "model.layers.1.mlp.gate (layer=1 not in layers=[7])" in rep.skipped
    _, rep = quantize_model(m, spec, names={"model.layers.9.mlp.gate"})
    assert "model.layers.0.mlp.gate (not in names=)" in rep.skipped
    d = rep.to_dict()
    assert d["realized_bytes_total"] == 0 and d["skipped_linear_count"] == len(rep.skipped)
    assert d["spec"]["names"] == ["model.layers.9.mlp.gate"] and d["padding"]["inflation_pct"] == 0.0
    assert set_dequant_mode(m, "separate") == 0 and reset_dequant_counters(m) == 0
    assert supported_dequant_modes(m) == ("separate",)
    with pytest.raises(ValueError):
        set_dequant_mode(m, "magic")


def _packed_cpu():
    codes = torch.randint(-127, 128, (16, 128), dtype=torch.int8)
    scale = torch.full((16, 1), 0.01, dtype=torch.float16)
    return QuantLinear.from_packed(codes, scale, in_features=128, group_size=128, name="x")


def test_dispatch_reasons_counters_and_no_cpu_arm():
    ql = _packed_cpu()
    x = torch.randn(1, 128, dtype=torch.float16)
    assert ql._fused_fallback_reason(x) == "not_cuda"
    set_dequant_mode(ql, "separate")
    assert ql._fused_fallback_reason(x) == "mode_is_separate"
    set_dequant_mode(ql, "fused")
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ql(x)  # no CPU arm: loud, and nothing counted
    act = dequant_activity(ql)
    assert (act["n_quant_linear"], act["modes"], act["fused_calls"], act["separate_calls"], act["fallbacks"]) == (
        1, {"fused": 1}, 0, 0, {})
    rb = realized_bytes(ql)
    assert rb == {"packed_bytes": 16 * 128, "scale_bytes": 32, "zero_bytes": 0, "bias_bytes": 0,
                  "total_bytes": 16 * 128 + 32}
