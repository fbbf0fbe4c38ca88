"""GPU parity of the two quantising operators that only wrapped other kernels
in their previous tests: ``QuantLinear`` and ``quantize_fused_experts``.

* ``QuantLinear`` (reference ``src/lemoq/quant/linear.py:245-488``) against the
  oracle, as the reference's K1 gate does (``tests/test_kernel_parity.py:134-220``):
  its buffers equal the oracle's RTN of the same weight bit for bit; one token
  (the fused arm, ``_fused_forward`` ``:446-469``) is within the K1 gate of the
  fp64 product (error <= 1.5 x the fp32 separate arm's) and the fp16
  tolerance rtol 2e-2 / atol 2e-3; seven tokens (the separate arm, ``:471-480``: fp16 dequantised
  weight, ``F.linear``) lie within one fp16 ulp of the fp64 product of the fp16
  weight plus the fp32 accumulation allowance 3e-5 * sum|x||w|.
* ``quantize_fused_experts`` on the device (reference
  ``src/lemoq/kernels/moe_grouped_quant.py:191-244``): fusing then quantising
  equals quantising each expert's gate, up and down matrices on their own
  with the oracle's RTN, bit for bit (``tests/test_moe_grouped_quant.py:76-114``).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close, assert_gate, randn
from oracle import ops
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def _ulp16(r: torch.Tensor) -> torch.Tensor:
    a = r.double().abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


@pytest.mark.parametrize("n,k,group", [(1024, 2048, 128), (300, 500, 128), (2048, 1024, 64)])
def test_quant_linear_buffers_equal_oracle_rtn(n, k, group, dev):
    from lemoq.quant.linear import QuantLinear

    print("case: QuantLinear buffers n=%d k=%d g=%d" % (n, k, group), flush=True)
    w = randn(n, k, seed=n + k, std=0.02)
    lin = QuantLinear(w.to(dev), group_size=group)
    ref = oq.rtn_quantize_w8(w.numpy(), group)
    assert np.array_equal(lin.packed.cpu().numpy(), ref["codes_padded"])
    assert np.array_equal(lin.scale.cpu().numpy().view(np.uint16), ref["scale_f16"].view(np.uint16))
    assert lin.padded_in == ref["codes_padded"].shape[1]


@pytest.mark.parametrize("n,k", [(1024, 2048), (2048, 2048), (300, 500)])
def test_quant_linear_one_token_vs_oracle(n, k, dev):
    """The fused arm against the fp64 product of x and code * fp16 scale."""
    from lemoq.quant.linear import QuantLinear

    print("case: QuantLinear M=1 n=%d k=%d" % (n, k), flush=True)
    w = randn(n, k, seed=7 * n + k, std=0.02)
    lin = QuantLinear(w.to(dev))
    codes, scale = lin.packed.cpu(), lin.scale.cpu()
    x = randn(1, k, seed=k + 3).to(torch.float16)
    got = lin(x.to(dev))
    torch.cuda.synchronize()
    assert got.shape == (1, n) and got.dtype == torch.float16
    wd = ops.dequant_w8(codes, scale, 128)[:, :k].double()
    oracle64 = x.double() @ wd.t()
    separate = ops.dequant_gemm_separate(x, codes, scale, 128, out_dtype=torch.float16)
    assert_gate(got, oracle64, separate, what="QuantLinear M=1 %dx%d" % (n, k))


@pytest.mark.parametrize("n,k", [(1024, 2048), (2048, 1024), (300, 500)])
def test_quant_linear_seven_tokens_vs_oracle(n, k, dev):
    """The multi-token arm against F.linear of the fp16 dequantised weight."""
    from lemoq.quant.linear import QuantLinear

    print("case: QuantLinear M=7 n=%d k=%d" % (n, k), flush=True)
    w = randn(n, k, seed=5 * n + k, std=0.02)
    lin = QuantLinear(w.to(dev))
    codes, scale = lin.packed.cpu(), lin.scale.cpu()
    x = randn(1, 7, k, seed=k + 4).to(torch.float16)
    got = lin(x.to(dev))
    torch.cuda.synchronize()
    assert got.shape == (1, 7, n) and got.dtype == torch.float16
    g = got.reshape(7, n).double().cpu()
    ref = ops.linear_separate_w8(x.reshape(7, k), codes, scale, 128)
    w16 = ops.dequant_weight_f16(codes, scale, 128)[:, :k].double()
    absdot = x.reshape(7, k).double().abs() @ w16.abs().t()
    bound = _ulp16(ref) + 3e-5 * absdot
    err = (g - ref.double()).abs()
    assert bool((err <= bound).all()), "max err %.3e, worst excess %.3e" % (float(err.max()), float((err - bound).max()))
    assert_close(got.reshape(7, n), ref, what="QuantLinear M=7")


@pytest.mark.parametrize("e,f,h,group", [(8, 256, 512, 32), (4, 1024, 2048, 128), (3, 96, 128, 32)])
def test_quantize_fused_experts_equals_per_expert_rtn(e, f, h, group, dev):
    from lemoq.kernels.moe_grouped_quant import FusedExperts, quantize_fused_experts

    print("case: quantize_fused_experts e=%d f=%d h=%d g=%d" % (e, f, h, group), flush=True)
    gate = randn(e, f, h, seed=e * f + h, std=0.02)
    up = randn(e, f, h, seed=e * f + h + 1, std=0.02)
    down = randn(e, h, f, seed=e * f + h + 2, std=0.02)
    # an all-zero group and exact half-way values exercise the scale-1.0 and tie rules
    gate[0, 0, :group] = 0.0
    up[-1, 1, :group] = 0.5 + torch.arange(group, dtype=torch.float32) - group // 2
    up[-1, 1, 0] = 127.0
    fused = FusedExperts(gate_up=torch.cat([gate, up], 1).to(dev), down=down.to(dev))
    q = quantize_fused_experts(fused, bits=8, group_size=group)
    torch.cuda.synchronize()
    assert tuple(q.packed_gate_up.shape) == (e, 2 * f, h) and tuple(q.packed_down.shape) == (e, h, f)
    for i in range(e):
        cases = (
            ("gate", gate[i], q.packed_gate_up[i, :f], q.scale_gate_up[i, :f]),
            ("up", up[i], q.packed_gate_up[i, f:], q.scale_gate_up[i, f:]),
            ("down", down[i], q.packed_down[i], q.scale_down[i]),
        )
        for name, wt, packed, scale in cases:
            ref = oq.rtn_quantize_w8(wt.numpy(), group)
            assert np.array_equal(packed.cpu().numpy(), ref["codes_padded"]), (i, name)
            assert np.array_equal(scale.cpu().numpy().view(np.uint16), ref["scale_f16"].view(np.uint16)), (i, name)
