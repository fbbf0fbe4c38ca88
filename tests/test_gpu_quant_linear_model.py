"""The QuantLinear surface over a whole model on the GPU: ``quantize_model``
on a module tree named like HF OLMoE (the reference's
``src/lemoq/quant/linear.py:592-694``), its report, the dispatch counters
(``dequant_activity``, ``set_dequant_mode``, ``reset_dequant_counters``,
``supported_dequant_modes``: ``:113-125,529-589``) and the fallback reasons
of ``_fused_fallback_reason`` (``:420-444``), and fp32 activations through both
arms against fp64 (rtol 2e-2 / atol 2e-3, the reference's fp16 tolerance)."""

from __future__ import annotations

import pytest
import torch
from torch import nn

from lemoq.quant.linear import (
    QuantLinear,
    SchemeSpec,
    dequant_activity,
    quantize_model,
    realized_bytes,
    reset_dequant_counters,
    set_dequant_mode,
    supported_dequant_modes,
)

pytestmark = pytest.mark.gpu

H, E = 256, 4


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
            setattr(self, n, nn.Linear(H, H, bias=False))


class _Expert(nn.Module):
    def __init__(self):
        super().__init__()
        self.gate_proj = nn.Linear(H, 128, bias=False)
        self.up_proj = nn.Linear(H, 128, bias=False)
        self.down_proj = nn.Linear(128, H, bias=False)


class _Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn = _Attn()
        self.mlp = nn.Module()
        self.mlp.gate = nn.Linear(H, E, bias=False)
        self.mlp.experts = nn.ModuleList([_Expert() for _ in range(E)])


def _model(dev):
    torch.manual_seed(0)
    m = nn.Module()
    m.model = nn.Module()
    m.model.embed_tokens = nn.Embedding(64, H)
    m.model.layers = nn.ModuleList([_Layer(), _Layer()])
    m.lm_head = nn.Linear(H, 320, bias=True)
    return m.to(dev)


def test_quantize_model_report_and_dispatch_counts(dev):
    print("case: quantize_model over an OLMoE-named tree, counters", flush=True)
    m = _model(dev)
    spec = SchemeSpec.from_flags("w8a16", 128, targets=("attention", "experts", "router", "lm_head"),
                                 keep_lm_head_fp16=True)
    _, rep = quantize_model(m, spec)
    assert rep.replaced == {"attention": 8, "experts": 24, "router": 2}
    assert rep.skipped == ["lm_head (keep_lm_head_fp16=True)"] and isinstance(m.lm_head, nn.Linear)
    qls = [q for q in m.modules() if isinstance(q, QuantLinear)]
    assert len(qls) == 34 and all(q.name for q in qls)
    d = rep.to_dict()
    assert d["realized_bytes_total"] == sum(realized_bytes(q)["total_bytes"] for q in qls)
    assert rep.realized_by_target["router"]["n_linear"] == 2 and d["padding"]["inflation_pct"] == 0.0
    # the router gate (4 x 256): its packed codes and scales are what it stores
    assert realized_bytes(m.model.layers[0].mlp.gate)["packed_bytes"] == E * H
    assert supported_dequant_modes(m) == ("separate", "fused")
    assert reset_dequant_counters(m) == 34
    q = m.model.layers[0].self_attn.q_proj
    x1 = torch.randn(1, H, device=dev).to(torch.float16)
    x3 = torch.randn(1, 3, H, device=dev).to(torch.float16)
    y1, y3 = q(x1), q(x3)
    assert y1.shape == (1, H) and y3.shape == (1, 3, H)
    act = dequant_activity(m)
    assert (act["fused_calls"], act["separate_calls"], act["fallbacks"]) == (1, 1, {"multi_token": 1})
    assert set_dequant_mode(m, "separate") == 34
    q(x1)
    act = dequant_activity(m)
    assert act["modes"] == {"separate": 34} and act["separate_calls"] == 2 and act["fallbacks"] == {"multi_token": 1}
    set_dequant_mode(m, "fused")
    assert q._fused_fallback_reason(x1.to(torch.bfloat16)) == "dtype_unsupported(bfloat16)"
    with pytest.raises(NotImplementedError):
        q(x1.to(torch.bfloat16))  # the separate arm has no bf16 GEMM here: refused, not guessed
    assert dequant_activity(m)["separate_calls"] == 2  # nothing counted for the refused call
    # a layer filter and the lm_head once keep_lm_head_fp16 is off, on a fresh tree
    m2 = _model(dev)
    spec2 = SchemeSpec.from_flags("w4a16", 128, targets=("lm_head", "router"), keep_lm_head_fp16=False)
    _, rep2 = quantize_model(m2, spec2, layers=[1])
    assert rep2.replaced == {"router": 1} and isinstance(m2.model.layers[1].mlp.gate, QuantLinear)
    assert "lm_head (layer=None not in layers=[1])" in rep2.skipped


@pytest.mark.parametrize("scheme,sym", [("w8a16", True), ("w4a16", False), ("mxfp4", True)])
def test_fp32_activations_through_both_arms(scheme, sym, dev):
    """fp32 x: one token takes the fused arm (the fp32-activation GEMV), three
    tokens the separate arm (fp32 weight products over the rows); both against
    fp64 on the dequantised weight, and the output stays fp32."""
    print("case: QuantLinear %s sym=%s fp32 activations" % (scheme, sym), flush=True)
    g = torch.Generator().manual_seed(5)
    w = torch.randn(192, 300, generator=g) * 0.05
    ql = QuantLinear(w.to(dev), group_size=64, scheme=scheme, symmetric=sym)
    w64 = ql.dequantized_weight().double().cpu()
    for rows in (1, 3):
        x = torch.randn(rows, 300, generator=g)
        reset_dequant_counters(ql)
        y = ql(x.to(dev))
        assert y.dtype == torch.float32
        act = dequant_activity(ql)
        assert act["fused_calls"] == (1 if rows == 1 else 0)
        ref = x.double() @ w64.T
        assert torch.allclose(y.double().cpu(), ref, rtol=2e-2, atol=2e-3), float((y.double().cpu() - ref).abs().max())
        assert float((y.double().cpu() - ref).abs().max()) < 1e-4  # fp32 products, fp32 sums


def test_install_packed_qkv_over_a_quantised_model(dev):
    """install_packed_qkv (the reference's ``packed_qkv.py:104-170``) on the
    quantised tree: one packed state per attention module, its projection
    bitwise equal to the three QuantLinear calls; counted and removed."""
    from lemoq.kernels.packed_qkv import install_packed_qkv, packed_qkv_installed, remove_packed_qkv

    print("case: install_packed_qkv", flush=True)
    m = _model(dev)
    with pytest.raises(ValueError, match="quantized q_proj"):
        install_packed_qkv(m)  # plain linears: refused, not silently three calls
    quantize_model(m, SchemeSpec.from_flags("w8a16", 128))
    assert install_packed_qkv(m) == 2 and packed_qkv_installed(m) == 2
    at = m.model.layers[1].self_attn
    x = torch.randn(1, H, device=dev).to(torch.float16)
    q, k, v = at._lemoq_packed_qkv.project(x)
    for got, proj in ((q, at.q_proj), (k, at.k_proj), (v, at.v_proj)):
        assert torch.equal(got, proj(x))
    assert remove_packed_qkv(m) == 2 and packed_qkv_installed(m) == 0
