"""GPU parity of the weight formats beyond 8-bit symmetric (8-bit asymmetric,
4-bit symmetric / asymmetric, MXFP4) and of the w8a8 activation fake-quant,
through the C-ABI wrappers.

- Quantisers (``lemoq_rtn_quantize``, ``lemoq_mxfp4_quantize``): codes,
  scales and zero points bit-exact to the oracle (``oracle.quant``), on the
  reference's case grid (``tests/test_quant_oracle.py:104-146``,
  ``tests/test_mxfp4.py``) and edge values (all-zero, largest and smallest
  normal weights, amax just below powers of two).
- Dequantisation (``lemoq_dequant_q``): fp32 weights bit-exact to the
  oracle's ``dequant_tile`` / ``mxfp4_dequantize`` (every E2M1 code at several
  scales, the -0 of code 8 included), fp16 weights their single rounding.
- Decode GEMV (``lemoq_gemv_q`` through ``dequant_gemm_fused``): the
  reference's K1 gate (``tests/test_kernel_parity.py:134-227``,
  ``tests/test_mxfp4_gpu.py``): within atol / rtol 1e-3 of the separate
  reference ``x @ dequant(w).T`` in fp32, and the A6 conjunction against an
  fp64 oracle (the kernel's error at most 1.5x the separate reference's).
  Cases: m = 1 and 4, K = 2048 / 256 / 500 / 50, groups 32-128, fp16 and fp32
  scales.
- ``QuantLinear`` per scheme, one token (fused arm) and several (separate arm).
- 4-bit grouped MoE (``lemoq_moe_gate_up_w4`` / ``lemoq_moe_down_w4`` through
  ``grouped_moe_forward_quant``): ``quantize_fused_experts(bits=4)`` bit-exact
  to the oracle's RTN and packing, the output against the oracle's grouped
  MoE on the unpacked codes and the fp64 closed form, the residual add and an
  out-of-range expert id.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import randn
from oracle import quant as oq

pytestmark = pytest.mark.gpu

TOL = dict(atol=1e-3, rtol=1e-3)


def _bits16(a) -> np.ndarray:
    return np.asarray(a).astype(np.float16).view(np.uint16)


def _rtn_vs_oracle(w: torch.Tensor, bits: int, group: int, sym: bool, dev):
    from lemoq.quant.rtn import quantize_rtn

    got = quantize_rtn(w.to(dev), bits=bits, group_size=group, symmetric=sym)
    ref = oq.rtn_quantize(w.numpy(), bits, group, sym)
    codes = got["codes_padded"].cpu().numpy().astype(np.int32)
    assert np.array_equal(codes, ref["codes_padded"]), "codes"
    assert np.array_equal(got["scale"].cpu().numpy(), ref["scale"]), "scale"
    assert np.array_equal(got["zero"].cpu().numpy(), ref["zero"]), "zero"
    assert np.array_equal(got["scale_f16"].cpu().numpy().view(np.uint16), _bits16(ref["scale"])), "scale fp16"
    assert np.array_equal(got["zero_f16"].cpu().numpy().view(np.uint16), _bits16(ref["zero"])), "zero fp16"
    if bits == 4:
        assert np.array_equal(got["packed"].cpu().numpy(), oq.pack_4bit(ref["codes_padded"])), "packed bytes"
    return got, ref


RTN_CASES = [(4, 128, True), (4, 32, True), (8, 64, True), (8, 128, True), (4, 128, False), (4, 64, False),
             (8, 128, False), (8, 32, False)]


@pytest.mark.parametrize("bits,group,sym", RTN_CASES)
@pytest.mark.parametrize("shape,seed", [((64, 2048), 0), ((64, 500), 1), ((3, 130), 7), ((1, 1), 2026)])
def test_rtn_quantize_bit_exact(bits, group, sym, shape, seed, dev):
    print("case: rtn bits=%d group=%d sym=%s shape=%s" % (bits, group, sym, shape), flush=True)
    _rtn_vs_oracle(randn(*shape, seed=seed, std=0.05), bits, group, sym, dev)


@pytest.mark.parametrize("fill", [0.0, float(np.finfo(np.float32).max), float(np.finfo(np.float32).tiny)],
                         ids=["zeros", "finfo_max", "finfo_tiny"])
@pytest.mark.parametrize("bits,group,sym", [(4, 128, True), (8, 32, True), (4, 128, False), (8, 32, False)])
def test_rtn_quantize_edge_values(fill, bits, group, sym, dev):
    print("case: rtn edge fill=%g bits=%d sym=%s" % (fill, bits, sym), flush=True)
    _rtn_vs_oracle(torch.full((16, 40), fill), bits, group, sym, dev)


def _mx_edge_rows() -> np.ndarray:
    rows = []
    for k in range(-20, 21):
        a = np.float32(2.0 ** k)
        for _ in range(5):
            a = np.nextafter(a, np.float32(0))
            blk = np.zeros(32, np.float32)
            blk[3], blk[7] = a, -a * np.float32(0.3)
            rows.append(blk)
    ties = np.zeros(32, np.float32)
    ties[:8] = [0.25, -0.25, 1.25, 2.5, -3.5, 5.0, 0.75, -1.75]
    rows.append(ties)
    return np.stack(rows)


@pytest.mark.parametrize("which", ["random", "wide", "padded", "edges", "zeros", "tiny"])
def test_mxfp4_quantize_bit_exact(which, dev):
    from lemoq.quant.mxfp4 import quantize_mxfp4

    print("case: mxfp4 quantize %s" % which, flush=True)
    w = {
        "random": lambda: randn(64, 256, seed=0, std=0.3).numpy(),
        "wide": lambda: randn(512, 2048, seed=3, std=0.05).numpy(),
        "padded": lambda: randn(4, 50, seed=3, std=0.2).numpy(),
        "edges": _mx_edge_rows,
        "zeros": lambda: np.zeros((2, 70), np.float32),
        "tiny": lambda: (randn(8, 64, seed=5, std=1.0) * 1e-30).numpy(),
    }[which]()
    got = quantize_mxfp4(torch.from_numpy(w).to(dev))
    ref = oq.mxfp4_quantize(w)
    assert got["padded_in"] == ref["padded_in"]
    assert np.array_equal(got["scales"].cpu().numpy(), ref["scales"]), "scale bytes"
    assert np.array_equal(got["codes_packed"].cpu().numpy(), ref["codes_packed"]), "codes"


@pytest.mark.parametrize("bits,group,sym", RTN_CASES)
@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_dequant_bit_exact(bits, group, sym, scale_dtype, dev):
    from lemoq.quant.formats import dequantize, format_id

    print("case: dequant bits=%d group=%d sym=%s scale %s" % (bits, group, sym, scale_dtype), flush=True)
    w = randn(40, 300, seed=bits * group, std=0.05)
    q = oq.rtn_quantize(w.numpy(), bits, group, sym)
    scale = torch.from_numpy(q["scale"]).to(scale_dtype)
    zero = torch.from_numpy(q["zero"]).to(scale_dtype)
    codes = q["codes_padded"]
    packed = torch.from_numpy(oq.pack_4bit(codes) if bits == 4 else
                              codes.astype(np.int8 if sym else np.uint8))
    ref = oq.dequant_tile(codes, scale.float().numpy(), zero.float().numpy(), group, sym, in_features=300)
    fmt = format_id(bits, sym)
    got32 = dequantize(packed.to(dev), scale.to(dev), None if sym else zero.to(dev), fmt=fmt, group_size=group,
                       k_out=300, dtype=torch.float32).cpu().numpy()
    assert np.array_equal(got32.view(np.uint32), ref.view(np.uint32))
    got16 = dequantize(packed.to(dev), scale.to(dev), None if sym else zero.to(dev), fmt=fmt, group_size=group,
                       k_out=300, dtype=torch.float16).cpu().numpy()
    assert np.array_equal(got16.view(np.uint16), _bits16(ref))


def test_mxfp4_dequant_every_code_and_scale(dev):
    """All 16 E2M1 codes (code 8 is -0) at scale bytes 0, 1, 100, 126, 127, 128,
    200, 254: fp32 bit-exact to the oracle, fp16 its one rounding."""
    from lemoq.quant.mxfp4 import dequantize_packed

    print("case: mxfp4 dequant table", flush=True)
    codes = np.tile(np.arange(16, dtype=np.uint8), (8, 4))  # 8 rows x 64 codes
    scales = np.repeat(np.array([[0], [1], [100], [126], [127], [128], [200], [254]], np.uint8), 2, axis=1)
    packed = oq.pack_4bit(codes)
    ref = oq.mxfp4_dequantize(packed, scales, 64)
    got = dequantize_packed(torch.from_numpy(packed).to(dev), torch.from_numpy(scales).to(dev), 64,
                            dtype=torch.float32).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    got16 = dequantize_packed(torch.from_numpy(packed).to(dev), torch.from_numpy(scales).to(dev), 64,
                              dtype=torch.float16).cpu().numpy()
    assert np.array_equal(got16.view(np.uint16), _bits16(ref))


def _gemv_case(m, k, n, bits, group, sym, *, scale_dtype=torch.float16, mxfp4=False, seed=0, dev="cuda",
               x32=False):
    """The reference's K1 gate for one case; returns (err_kernel, err_ref).
    ``x32``: fp32 activations (``lemoq_gemv_q_x32``), not rounded to fp16."""
    from lemoq.kernels.dequant_gemm import dequant_gemm_fused

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g) * 0.5
    x = x if x32 else x.to(torch.float16)
    w = torch.randn(n, k, generator=g) * 0.05
    if mxfp4:
        q = oq.mxfp4_quantize(w.numpy())
        packed = torch.from_numpy(q["codes_packed"])
        scale = torch.from_numpy(q["scales"])
        zero = None
        w_ref = torch.from_numpy(oq.mxfp4_dequantize(q["codes_packed"], q["scales"], k))
        w64 = w_ref.double()
        group = 32
    else:
        q = oq.rtn_quantize(w.numpy(), bits, group, sym)
        codes = q["codes_padded"]
        packed = torch.from_numpy(oq.pack_4bit(codes) if bits == 4 else codes.astype(np.int8 if sym else np.uint8))
        scale = torch.from_numpy(q["scale"]).to(scale_dtype)
        zero = torch.from_numpy(q["zero"]).to(scale_dtype)
        w_ref = torch.from_numpy(oq.dequant_tile(codes, scale.float().numpy(), zero.float().numpy(), group, sym,
                                                 in_features=k))
        w64 = torch.from_numpy(oq.dequant_tile(codes, q["scale"], q["zero"], group, sym, in_features=k)).double()
    ref = x.float() @ w_ref.T  # the separate reference (fp32)
    got = dequant_gemm_fused(x.to(dev), packed.to(dev), scale.to(dev),
                             None if (sym or mxfp4) else zero.to(dev), group_size=group,
                             bits=4 if mxfp4 else bits, symmetric=sym, out_dtype=torch.float32,
                             mxfp4=mxfp4).cpu()
    assert torch.allclose(got, ref, **TOL), float((got - ref).abs().max())
    oracle = x.double() @ w64.T
    err_ref = float((ref.double() - oracle).abs().max())
    err_got = float((got.double() - oracle).abs().max())
    # with fp32 activations both errors are fp32 summation noise (1e-7 on these
    # outputs) and their ratio is chance, so the gate gets a floor of 1e-6 there
    floor = 1e-6 * max(1.0, float(oracle.abs().max())) if x32 else 1e-9
    assert err_got <= 1.5 * err_ref + floor, (err_got, err_ref)
    return err_got, err_ref


GEMV_CASES = [
    # (m, k, n, bits, group, sym, scale dtype): the reference's K1 grid plus the asymmetric formats
    (1, 2048, 2048, 8, 128, True, torch.float16), (1, 2048, 2048, 4, 128, True, torch.float16),
    (4, 256, 512, 8, 128, True, torch.float16), (4, 256, 512, 4, 128, True, torch.float16),
    (1, 512, 256, 8, 128, True, torch.float32), (1, 512, 256, 4, 128, True, torch.float32),
    (1, 500, 256, 8, 128, True, torch.float16), (1, 500, 256, 4, 128, True, torch.float16),
    (1, 1024, 512, 8, 64, True, torch.float16), (1, 1024, 512, 4, 32, True, torch.float16),
    (1, 2048, 2048, 8, 128, False, torch.float16), (1, 2048, 2048, 4, 128, False, torch.float16),
    (4, 256, 512, 8, 128, False, torch.float16), (4, 256, 512, 4, 64, False, torch.float16),
    (1, 500, 256, 4, 128, False, torch.float32), (1, 8192, 64, 4, 128, True, torch.float16),
    (1, 8192, 64, 8, 128, False, torch.float16), (3, 4096, 300, 4, 128, False, torch.float16),
]


@pytest.mark.parametrize("m,k,n,bits,group,sym,sd", GEMV_CASES)
def test_gemv_formats_k1_gate(m, k, n, bits, group, sym, sd, dev):
    print("case: gemv m=%d k=%d n=%d bits=%d group=%d sym=%s scale %s" % (m, k, n, bits, group, sym, sd),
          flush=True)
    _gemv_case(m, k, n, bits, group, sym, scale_dtype=sd, seed=m * k + n + bits, dev=dev)


@pytest.mark.parametrize("m,k,n,bits,group,sym,sd", GEMV_CASES + [(1, 8192, 64, 8, 128, True, torch.float16),
                                                                  (1, 4098, 40, 8, 64, True, torch.float16),
                                                                  (2, 4098, 40, 4, 64, False, torch.float16)])
def test_gemv_formats_fp32_activations_k1_gate(m, k, n, bits, group, sym, sd, dev):
    """The reference's operator takes fp32 x as well (``_dequant_triton.py:252``):
    the fp32-activation kernel against the fp32 separate reference and fp64 on
    every case of the fp16 grid, plus K values that leave a ragged tail (4098,
    whose x rows also miss the 16-byte vector path) and the widest rows (8192)."""
    print("case: gemv fp32 x m=%d k=%d n=%d bits=%d group=%d sym=%s scale %s" % (m, k, n, bits, group, sym, sd),
          flush=True)
    _gemv_case(m, k, n, bits, group, sym, scale_dtype=sd, seed=m * k + n + bits + 1, dev=dev, x32=True)


@pytest.mark.parametrize("m,k,n,seed", [(1, 256, 128, 0), (3, 2048, 512, 3), (1, 50, 128, 2)])
def test_gemv_mxfp4_fp32_activations_k1_gate(m, k, n, seed, dev):
    print("case: gemv mxfp4 fp32 x m=%d k=%d n=%d" % (m, k, n), flush=True)
    _gemv_case(m, k, n, 4, 32, True, mxfp4=True, seed=seed + 50, dev=dev, x32=True)


@pytest.mark.parametrize("m,k,n,seed", [(1, 256, 128, 0), (4, 256, 128, 1), (1, 50, 128, 2), (1, 2048, 512, 3),
                                        (1, 2048, 2048, 7), (2, 8192, 96, 9)])
def test_gemv_mxfp4_k1_gate(m, k, n, seed, dev):
    print("case: gemv mxfp4 m=%d k=%d n=%d" % (m, k, n), flush=True)
    _gemv_case(m, k, n, 4, 32, True, mxfp4=True, seed=seed, dev=dev)


def test_gemv_w8_sym_fp32_scale_equals_fp16_path_on_exact_scales(dev):
    """The generic kernel (fp32 scales) and the decode step's w8 GEMV (fp16
    scales) on the same fp16-representable scales: equal up to the fp32 order."""
    from lemoq.kernels.dequant_gemm import dequant_gemm_fused

    print("case: w8 fp32-scale vs fp16-scale paths", flush=True)
    x = randn(1, 2048, seed=1, std=0.5).to(torch.float16).to(dev)
    q = oq.rtn_quantize(randn(1024, 2048, seed=2, std=0.05).numpy(), 8, 128, True)
    codes = torch.from_numpy(q["codes_padded"].astype(np.int8)).to(dev)
    s16 = torch.from_numpy(q["scale"]).half().to(dev)
    a = dequant_gemm_fused(x, codes, s16, group_size=128, bits=8)
    b = dequant_gemm_fused(x, codes, s16.float(), group_size=128, bits=8)
    assert torch.allclose(a, b, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("scheme,sym", [("w4a16", True), ("w4a16", False), ("w8a16", False), ("mxfp4", True),
                                        ("w8a8", True), ("w8a16", True)])
def test_quant_linear_schemes(scheme, sym, dev):
    """One token through the fused arm and five through the separate arm, each
    against its reference: fused = x @ dequant(w).T in fp32 (K1 tolerance),
    separate = fp16(x @ fp16(dequant(w)).T) (fp16 GEMM tolerance); w8a8 also
    checks the per-token fake-quant bit for bit."""
    from lemoq.quant.linear import QuantLinear

    print("case: QuantLinear %s sym=%s" % (scheme, sym), flush=True)
    w = randn(384, 512, seed=31, std=0.05)
    bias = randn(384, seed=32, std=0.1).to(torch.float16)
    ql = QuantLinear(w.to(dev), group_size=128, bias=bias.to(dev), scheme=scheme, symmetric=sym)
    if scheme == "mxfp4":
        assert ql.group_size == 32 and ql.scale.dtype == torch.uint8 and ql.zero is None
        q = oq.mxfp4_quantize(w.numpy())
        assert np.array_equal(ql.packed.cpu().numpy(), q["codes_packed"])
        wdq = oq.mxfp4_dequantize(q["codes_packed"], q["scales"], 512)
    else:
        bits = 4 if scheme == "w4a16" else 8
        q = oq.rtn_quantize(w.numpy(), bits, 128, sym)
        wdq = oq.dequant_tile(q["codes_padded"], q["scale"].astype(np.float16).astype(np.float32),
                              q["zero"].astype(np.float16).astype(np.float32), 128, sym, in_features=512)
    wdq_t = torch.from_numpy(wdq)
    assert np.array_equal(ql.dequantized_weight().cpu().numpy().view(np.uint32), wdq.view(np.uint32))
    for T in (1, 5):
        x = randn(T, 512, seed=33 + T, std=0.5).to(torch.float16)
        xin = x
        if scheme == "w8a8":  # per-token int8 fake quant (src/lemoq/quant/linear.py:398-414)
            xf = x.float()
            amax = xf.abs().amax(-1, keepdim=True)
            s = torch.where(amax > 0, amax / 127.0, torch.ones_like(amax))
            xin = ((xf / s).round().clamp(-128, 127) * s).to(torch.float16)
            got_fq = ql._fake_quant_activation(x.to(dev)).cpu()
            assert torch.equal(got_fq.view(torch.int16), xin.view(torch.int16))
        y = ql(x.to(dev)).cpu()
        if T == 1:
            ref = (xin.float() @ wdq_t.T + bias.float())
            assert torch.allclose(y.float(), ref, atol=2e-3, rtol=2e-3), float((y.float() - ref).abs().max())
        else:
            ref = (xin.double() @ wdq_t.half().double().T).half().float() + bias.float()
            assert torch.allclose(y.float(), ref, atol=3e-3, rtol=3e-3), float((y.float() - ref).abs().max())


# ---------------------------------------------------------------------------
# 4-bit grouped MoE (grouped_moe_forward_quant on QuantFusedExperts(bits=4))
# ---------------------------------------------------------------------------
def _q4_experts(E, F, H, group, seed, dev):
    """fp experts quantised on the device with bits=4; checked bit for bit
    against the oracle's 4-bit RTN and packing, row block by row block."""
    from lemoq.kernels.moe_grouped_quant import FusedExperts, quantize_fused_experts

    gu = randn(E, 2 * F, H, seed=seed, std=0.02)
    dn = randn(E, H, F, seed=seed + 1, std=0.02)
    q = quantize_fused_experts(FusedExperts(gu.to(dev), dn.to(dev)), bits=4, group_size=group)
    assert q.bits == 4 and q.packed_gate_up.dtype == torch.uint8
    assert tuple(q.packed_gate_up.shape) == (E, 2 * F, H // 2) and tuple(q.packed_down.shape) == (E, H, F // 2)
    out = []
    for w, packed, scale in ((gu, q.packed_gate_up, q.scale_gate_up), (dn, q.packed_down, q.scale_down)):
        ref = oq.rtn_quantize(w.reshape(-1, w.shape[-1]).numpy(), 4, group, True)
        assert np.array_equal(packed.cpu().reshape(-1, w.shape[-1] // 2).numpy(), oq.pack_4bit(ref["codes_padded"]))
        assert np.array_equal(scale.cpu().reshape(-1, w.shape[-1] // group).numpy().view(np.uint16),
                              _bits16(ref["scale"]))
        out.append(torch.from_numpy(ref["codes_padded"].astype(np.int8)).reshape(w.shape))
        out.append(scale.cpu())
    return q, out  # out: int8 codes (-8..7) and fp16 scales of gate/up and down


@pytest.mark.parametrize("E,F,H,K,group", [(64, 1024, 2048, 8, 128), (8, 256, 512, 2, 128), (4, 256, 512, 2, 32),
                                           (16, 128, 1024, 4, 64)])
def test_grouped_moe_w4_vs_oracle_and_fp64(E, F, H, K, group, dev):
    """The reference's quantised grouped gate (``tests/test_kernel_parity.py:230-282``,
    8- and 4-bit): the oracle's grouped MoE on the unpacked int4 codes (same
    arithmetic as at 8 bits) and the fp64 closed form with the fp16 act
    rounding point."""
    from helpers import assert_close
    from lemoq.kernels.moe_grouped_quant import grouped_moe_forward_quant
    from oracle import ops

    print("case: grouped moe w4 E=%d F=%d H=%d K=%d group=%d" % (E, F, H, K, group), flush=True)
    q, (gc, gs, dc, ds) = _q4_experts(E, F, H, group, seed=E + F + group, dev=dev)
    x = randn(H, seed=3).to(torch.float16)
    ids = torch.randperm(E, generator=torch.Generator().manual_seed(4))[:K]
    w = torch.softmax(randn(K, seed=5), 0).to(torch.float16)
    got = grouped_moe_forward_quant(x.to(dev), q, ids.to(dev), w.to(dev)).cpu()
    ref, act_ref = ops.grouped_moe_w8(x, gc, gs, dc, ds, group, ids, w)
    gu64 = torch.stack([ops.dequant_w8(gc[e], gs[e], group) for e in ids.tolist()]).double()
    g = gu64[:, :F] @ x.double()
    u = gu64[:, F:] @ x.double()
    act64 = (g * torch.sigmoid(g) * u).to(torch.float16).double()
    dn64 = torch.stack([ops.dequant_w8(dc[e], ds[e], group) for e in ids.tolist()]).double()
    out64 = ((dn64 @ act64.unsqueeze(-1)).squeeze(-1) * w.double().unsqueeze(1)).sum(0)
    assert_close(got, out64, what="moe w4 vs fp64")
    assert_close(got, ref, what="moe w4 vs oracle")


def test_grouped_moe_w4_reference_case_residual_and_invalid_id(dev):
    """E=4, F=256, H=512, ids (0, 2), weights (0.7, 0.3) as the reference's gate;
    the residual add keeps the fp16 rounding point; an out-of-range expert id
    contributes nothing."""
    from lemoq.kernels.moe_grouped_quant import grouped_moe_forward_quant

    print("case: grouped moe w4 reference case", flush=True)
    q, _ = _q4_experts(4, 256, 512, 128, seed=0, dev=dev)
    x = (randn(512, seed=1) * 0.5).to(torch.float16).to(dev)
    ids = torch.tensor([0, 2], dtype=torch.int64, device=dev)
    wts = torch.tensor([0.7, 0.3], dtype=torch.float16, device=dev)
    y = grouped_moe_forward_quant(x, q, ids, wts)
    resid = randn(512, seed=2).to(torch.float16).to(dev)
    assert torch.equal(grouped_moe_forward_quant(x, q, ids, wts, residual=resid), y + resid)
    one = grouped_moe_forward_quant(x, q, ids[:1], wts[:1])
    bad = grouped_moe_forward_quant(x, q, torch.tensor([0, 99], device=dev), wts)
    assert torch.equal(bad, one)


def test_quant_fused_experts_w4_dequant_bit_exact(dev):
    from lemoq.kernels.moe_grouped_quant import FusedExperts, quantize_fused_experts

    print("case: QuantFusedExperts w4 dequant", flush=True)
    gu = randn(3, 256, 512, seed=11, std=0.02)
    dn = randn(3, 512, 128, seed=12, std=0.02)
    q = quantize_fused_experts(FusedExperts(gu.to(dev), dn.to(dev)), bits=4, group_size=64)
    for got, w, k in ((q.dequant_gate_up_expert(1), gu[1], 512), (q.dequant_down_expert(2), dn[2], 128)):
        r = oq.rtn_quantize(w.numpy(), 4, 64, True)
        ref = oq.dequant_tile(r["codes_padded"], r["scale"].astype(np.float16).astype(np.float32), None, 64, True)
        assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert tuple(q.dequant_gate_up(torch.float16).shape) == (3, 256, 512)
    # the module-level form (the reference's dequantize_fused_experts) is the same dequantisation
    from lemoq.kernels.moe_grouped_quant import dequantize_fused_experts

    f = dequantize_fused_experts(q)
    assert torch.equal(f.gate_up[1], q.dequant_gate_up_expert(1)) and torch.equal(f.down[2], q.dequant_down_expert(2))
    assert dequantize_fused_experts(q, torch.float16).down.dtype == torch.float16


@pytest.mark.parametrize("bits,sym", [(8, True), (8, False), (4, True), (4, False)])
def test_quantize_linear_api_and_quantization_error(bits, sym, dev):
    """``lemoq.quant.quantize_linear`` / ``dequantize_reference`` (the reference's
    ``api.py:91-171``) on the device: the dequantised weight is the oracle's
    dequantisation bit for bit, also when rebuilt from the unpacked codes alone;
    ``rtn.quantization_error`` reports errors within the rounding bound."""
    import lemoq.quant as lq
    from lemoq.quant.rtn import quantization_error

    print("case: quantize_linear bits=%d sym=%s" % (bits, sym), flush=True)
    w = randn(96, 300, seed=bits + (0 if sym else 1), std=0.05)
    ql = lq.quantize_linear(w.to(dev), bits=bits, group_size=64, symmetric=sym)
    assert ql.shape == (96, 300) and ql.meta["padded_in"] == 320 and ql.scheme == "rtn"
    got = lq.dequantize_reference(ql).cpu()
    r = oq.rtn_quantize(w.numpy(), bits, 64, sym)
    ref = oq.dequant_tile(r["codes_padded"], r["scale"], r["zero"], 64, sym, in_features=300)
    assert np.array_equal(got.numpy().view(np.uint32), ref.view(np.uint32))
    bare = lq.QuantizedLinear(codes=ql.codes, scale=ql.scale, zero=ql.zero, bits=bits, group_size=64, symmetric=sym,
                              scheme="rtn", shape=ql.shape, meta={"n_groups": 5, "padded_in": 320})
    assert torch.equal(lq.dequantize_reference(bare), lq.dequantize_reference(ql))
    q = {"packed": ql.meta["packed"], "scale": ql.scale, "zero": ql.zero, "bits": bits, "group_size": 64,
         "symmetric": sym, "shape": ql.shape}
    e = quantization_error(w.to(dev), q)
    step = float(ql.scale.max())
    assert e["max_abs_err"] <= (0.5 if sym else 1.0) * step * (1 + 1e-5) and e["mean_abs_err"] < e["max_abs_err"]
    assert e["snr_db"] > (30.0 if bits == 8 else 10.0)
    assert e["max_rel_err_vs_absmax"] == pytest.approx(e["max_abs_err"] / float(w.abs().max()), rel=1e-5)
