"""Host-side argument checks of the weight-format wrappers (no GPU needed):
``dequant_gemm_fused`` raises the reference's exception types before touching
a device (``src/lemoq/kernels/_dequant_triton.py:200-262``,
``tests/test_mxfp4_gpu.py:104-146``), and the scheme table of ``QuantLinear``
(``src/lemoq/quant/linear.py:76-110,140-190``)."""

from __future__ import annotations

import pytest
import torch


def _mx_args(k=256, n=64):
    packed = torch.zeros((n, k // 2), dtype=torch.uint8)
    scales = torch.full((n, k // 32), 127, dtype=torch.uint8)
    x = torch.zeros((1, k), dtype=torch.float16)
    return x, packed, scales


def test_mxfp4_argument_rejections():
    from lemoq.kernels.dequant_gemm import dequant_gemm_fused

    x, packed, scales = _mx_args()
    with pytest.raises(ValueError, match="uint8"):
        dequant_gemm_fused(x, packed, scales.half(), None, group_size=32, bits=4, mxfp4=True)
    with pytest.raises(ValueError, match="32"):
        dequant_gemm_fused(x, packed, torch.full((64, 2), 127, dtype=torch.uint8), None, group_size=128, bits=4,
                           mxfp4=True)
    with pytest.raises(ValueError, match="zero"):
        dequant_gemm_fused(x, packed, scales, torch.zeros_like(scales), group_size=32, bits=4, symmetric=False,
                           mxfp4=True)
    with pytest.raises(ValueError, match="4-bit"):
        dequant_gemm_fused(x, packed, scales, None, group_size=32, bits=8, mxfp4=True)


def test_format_argument_rejections():
    from lemoq.kernels.dequant_gemm import dequant_gemm_fused

    x = torch.zeros((1, 256), dtype=torch.float16)
    s = torch.ones((64, 2), dtype=torch.float16)
    with pytest.raises(ValueError, match="zero point"):  # asymmetric without zero
        dequant_gemm_fused(x, torch.zeros((64, 256), dtype=torch.uint8), s, None, group_size=128, bits=8,
                           symmetric=False)
    with pytest.raises(ValueError, match="uint8"):  # asymmetric 8-bit codes stored as int8
        dequant_gemm_fused(x, torch.zeros((64, 256), dtype=torch.int8), s, s, group_size=128, bits=8,
                           symmetric=False)
    with pytest.raises(ValueError, match="width"):  # 4-bit needs padded_in / 2 bytes per row
        dequant_gemm_fused(x, torch.zeros((64, 256), dtype=torch.uint8), s, None, group_size=128, bits=4)
    with pytest.raises(ValueError, match="exceeds"):
        dequant_gemm_fused(torch.zeros((1, 300), dtype=torch.float16), torch.zeros((64, 128), dtype=torch.uint8),
                           s, None, group_size=128, bits=4)
    with pytest.raises(NotImplementedError):
        dequant_gemm_fused(x, torch.zeros((64, 256), dtype=torch.int8), s, None, group_size=128, bits=6)
    with pytest.raises(NotImplementedError, match="group_size"):  # 4-bit groups must be whole 16-byte slices
        dequant_gemm_fused(x, torch.zeros((64, 128), dtype=torch.uint8), torch.ones((64, 16), dtype=torch.float16),
                           None, group_size=16, bits=4)
    with pytest.raises(NotImplementedError, match="fp16 or fp32"):  # fp32 x is taken, bf16 is not
        dequant_gemm_fused(x.bfloat16(), torch.zeros((64, 128), dtype=torch.uint8), s, None, group_size=128, bits=4)
    # bits inferred from the code dtype: uint8 -> 4-bit
    with pytest.raises(ValueError, match="width"):
        dequant_gemm_fused(x, torch.zeros((64, 256), dtype=torch.uint8), s, None, group_size=128)


def test_scheme_table():
    from lemoq.quant.linear import SchemeSpec, parse_scheme

    assert parse_scheme("w8a16") == (8, None) and parse_scheme("W4A16") == (4, None)
    assert parse_scheme("w8a8") == (8, 8) and parse_scheme("mxfp4") == (4, None) and parse_scheme("fp16") == (None, None)
    with pytest.raises(ValueError):
        parse_scheme("w3a16")
    spec = SchemeSpec.from_flags("mxfp4", 128, targets=("attention",))
    assert spec.group_size == 32 and spec.enabled
    assert not SchemeSpec.from_flags("fp16", 128).enabled
    with pytest.raises(ValueError):
        SchemeSpec.from_flags("w8a16", 128, dequant="sometimes")


def test_pack_4bit_torch_matches_the_reference_convention():
    from lemoq.quant.pack import bit_cost, pack_4bit, unpack_4bit

    c = torch.tensor([[1, -1, 7, -8]])
    assert pack_4bit(c).tolist() == [[0xF1, 0x87]]
    assert unpack_4bit(pack_4bit(c)).tolist() == c.tolist()
    assert unpack_4bit(torch.tensor([[0xF1]], dtype=torch.uint8), signed=False).tolist() == [[1, 15]]
    with pytest.raises(ValueError):
        pack_4bit(torch.zeros((2, 3), dtype=torch.int32))
    assert bit_cost(2 * 130, 4, 128, in_features=130)["scale_bytes"] == 2 * 2 * 2  # 2 rows x 2 groups x 2 B


def test_grouped_launch_plan_4bit_shapes():
    """Host-side plan of the 4-bit grouped MoE: packed widths halved, uint8 codes,
    group a multiple of the 32-code lane slice."""
    from lemoq.kernels.moe_grouped_quant import QuantFusedExperts, quant_launch_plan

    E, F, H, g = 8, 256, 512, 64
    q = QuantFusedExperts(torch.zeros((E, 2 * F, H // 2), dtype=torch.uint8),
                          torch.ones((E, 2 * F, H // g), dtype=torch.float16),
                          torch.zeros((E, H, F // 2), dtype=torch.uint8),
                          torch.ones((E, H, F // g), dtype=torch.float16), bits=4, group_size=g)
    assert q.hidden == H and q.ffn == F
    plan = quant_launch_plan(q, top_k=2)
    assert plan["kernels"] == ("lemoq_moe_gate_up_w4", "lemoq_moe_down_w4") and plan["quant"]["bits"] == 4
    bad = QuantFusedExperts(q.packed_gate_up.to(torch.int8), q.scale_gate_up, q.packed_down, q.scale_down, bits=4,
                            group_size=g)
    with pytest.raises(ValueError, match="uint8"):
        quant_launch_plan(bad, top_k=2)
    g16 = QuantFusedExperts(q.packed_gate_up, torch.ones((E, 2 * F, H // 16), dtype=torch.float16),
                            q.packed_down, torch.ones((E, H, F // 16), dtype=torch.float16), bits=4, group_size=16)
    with pytest.raises(ValueError, match="multiple of 32"):
        quant_launch_plan(g16, top_k=2)
