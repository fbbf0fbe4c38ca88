"""Pins of the floating-point CPU oracle (oracle/ops.py) — CPU only.

Independent checks: fp64 brute force on small shapes, closed forms and
invariants (split-count invariance, linearity, permutation of expert slots,
empty lengths, NaN tails), and the installed HF transformers OLMoE modules
(RMSNorm, rotary embedding, rotate_half RoPE) whose math the reference calls
at its boundary (transformers 4.57.6 there; the installed 5.15 code of these
functions is the same arithmetic).  Cases mirror the reference's
tests/test_attn_decode.py:74-149, tests/test_kv_int8.py:134-169,
tests/test_rmsnorm_parity.py:20-58, tests/test_fused_rope.py:114-143,
tests/test_kernel_parity.py:189, :256-282 of LeanMoE-Quant.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ops
from oracle import quant as oq


def _g(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------------------
# dense w8 GEMV
# ---------------------------------------------------------------------------
def test_dequant_gemm_vs_fp64_brute_force_loops():
    n, k, g = 6, 64, 32
    w = (torch.randn((n, k), generator=_g(1)) * 0.02).numpy()
    q = oq.rtn_quantize_w8(w, g)
    codes, scale = torch.from_numpy(q["codes_padded"]), torch.from_numpy(q["scale_f16"])
    x = torch.randn((2, k), generator=_g(2)).to(torch.float16)
    y = ops.dequant_gemm_separate(x, codes, scale, g)
    for m in range(2):
        for r in range(n):
            acc = 0.0
            for c in range(k):
                acc += float(x[m, c]) * int(codes[r, c]) * float(scale[r, c // g])
            assert abs(float(y[m, r]) - acc) <= 1e-5 * (1 + abs(acc))


@pytest.mark.parametrize("k", [2048, 500, 256])
def test_dequant_gemm_separate_equals_group_tiles(k):
    w = (torch.randn((96, k), generator=_g(k)) * 0.02).numpy()
    q = oq.rtn_quantize_w8(w, 128)
    codes, scale = torch.from_numpy(q["codes_padded"]), torch.from_numpy(q["scale_f16"])
    x = torch.randn((3, k), generator=_g(k + 1)).to(torch.float16)
    a = ops.dequant_gemm_separate(x, codes, scale, 128)
    b = ops.dequant_gemm_fused_tiles(x, codes, scale, 128)
    assert torch.allclose(a, b, rtol=1e-5, atol=1e-6)


def test_dequant_uses_the_fp16_scale():
    w = (torch.randn((4, 128), generator=_g(4)) * 0.02).numpy()
    q = oq.rtn_quantize_w8(w, 128)
    d = ops.dequant_w8(torch.from_numpy(q["codes_padded"]), torch.from_numpy(q["scale_f16"]), 128)
    expect = q["codes_padded"].astype(np.float32) * q["scale_f16"].astype(np.float32)
    assert np.array_equal(d.numpy(), expect)


# ---------------------------------------------------------------------------
# RMSNorm / RoPE against HF transformers (the reference's third-party boundary)
# ---------------------------------------------------------------------------
def _hf():
    return pytest.importorskip("transformers.models.olmoe.modeling_olmoe")


@pytest.mark.parametrize("rows,h", [(1, 2048), (16, 128), (3, 1000)])
def test_rms_norm_bitwise_equals_hf_olmoe_rmsnorm(rows, h):
    m = _hf()
    x = (torch.randn((rows, h), generator=_g(h)) * 3).to(torch.float16)
    w = (torch.rand((h,), generator=_g(h + 1)) + 0.5).to(torch.float16)
    ref = m.OlmoeRMSNorm(h, eps=1e-5)
    ref.weight.data = w.clone()
    with torch.no_grad():
        expect = ref(x)
    got = ops.rms_norm(x, w, 1e-5)
    assert got.dtype == torch.float16 and torch.equal(got, expect)


def test_rotary_tables_bitwise_equal_hf_rotary_embedding():
    m = _hf()
    from transformers.models.olmoe.configuration_olmoe import OlmoeConfig

    cfg = OlmoeConfig(hidden_size=2048, num_attention_heads=16, max_position_embeddings=4096, rope_theta=1e4)
    rot = m.OlmoeRotaryEmbedding(cfg)
    pos = torch.arange(0, 4096, 7).reshape(1, -1)
    x = torch.zeros((1, 1, 128), dtype=torch.float16)
    cos_hf, sin_hf = rot(x, pos)
    cos, sin = ops.rotary_cos_sin(pos.reshape(-1), 128, 1e4)
    assert torch.equal(cos, cos_hf[0]) and torch.equal(sin, sin_hf[0])


@pytest.mark.parametrize("pos", [0, 1, 1024, 4095])
def test_rope_fused_equals_hf_rotate_half_in_fp32(pos):
    m = _hf()
    cos, sin = ops.rotary_cos_sin(torch.tensor([pos]), 128, 1e4)
    q = torch.randn((16, 128), generator=_g(pos)).to(torch.float16)
    k = torch.randn((16, 128), generator=_g(pos + 1)).to(torch.float16)
    qh, kh = m.apply_rotary_pos_emb(q.float()[None], k.float()[None], cos.float(), sin.float(), unsqueeze_dim=0)
    assert torch.equal(ops.rope_fused(q, cos[0], sin[0]), qh[0].to(torch.float16))
    assert torch.equal(ops.rope_fused(k, cos[0], sin[0]), kh[0].to(torch.float16))
    # against fp64 rotation: within one fp16 rounding
    d = q.double()
    rot = torch.cat((-d[:, 64:], d[:, :64]), -1)
    ref = d * cos[0].double() + rot * sin[0].double()
    assert (ops.rope_fused(q, cos[0], sin[0]).double() - ref).abs().max() <= 2e-3 * ref.abs().max()


# ---------------------------------------------------------------------------
# grouped MoE
# ---------------------------------------------------------------------------
def _experts(E, F, H, seed):
    gu = (torch.randn((E * 2 * F, H), generator=_g(seed)) * 0.02).numpy()
    dn = (torch.randn((E * H, F), generator=_g(seed + 1)) * 0.02).numpy()
    qg, qd = oq.rtn_quantize_w8(gu, 128), oq.rtn_quantize_w8(dn, 128)
    return (torch.from_numpy(qg["codes_padded"]).reshape(E, 2 * F, H),
            torch.from_numpy(qg["scale_f16"]).reshape(E, 2 * F, H // 128),
            torch.from_numpy(qd["codes_padded"]).reshape(E, H, F),
            torch.from_numpy(qd["scale_f16"]).reshape(E, H, F // 128))


def test_grouped_moe_vs_fp64_closed_form():
    E, F, H, K = 8, 256, 512, 2
    gc, gs, dc, ds = _experts(E, F, H, 3)
    x = torch.randn((H,), generator=_g(5)).to(torch.float16)
    ids = torch.tensor([5, 1])
    tw = torch.tensor([0.7, 0.3]).to(torch.float16)
    out, act = ops.grouped_moe_w8(x, gc, gs, dc, ds, 128, ids, tw)
    ref = torch.zeros(H, dtype=torch.float64)
    for i, e in enumerate(ids.tolist()):
        wg = ops.dequant_w8(gc[e], gs[e], 128).double()
        wd = ops.dequant_w8(dc[e], ds[e], 128).double()
        gate, up = wg[:F] @ x.double(), wg[F:] @ x.double()
        a = (gate * torch.sigmoid(gate) * up).to(torch.float16).double()  # act rounded to fp16
        assert torch.allclose(act[i].double(), a, rtol=2e-3, atol=1e-5)
        ref += float(tw[i]) * (wd @ a)
    assert (out.double() - ref).abs().max() <= 1e-3 * (1 + ref.abs().max())


def test_grouped_moe_linear_in_weights_and_slot_order_free():
    E, F, H = 4, 128, 256
    gc, gs, dc, ds = _experts(E, F, H, 8)
    x = torch.randn((H,), generator=_g(9)).to(torch.float16)
    ids = torch.tensor([3, 0, 2])
    tw = torch.tensor([0.5, 0.25, 0.125]).to(torch.float16)
    a, _ = ops.grouped_moe_w8(x, gc, gs, dc, ds, 128, ids, tw)
    b, _ = ops.grouped_moe_w8(x, gc, gs, dc, ds, 128, ids.flip(0), tw.flip(0))
    assert torch.allclose(a.float(), b.float(), atol=2e-3, rtol=1e-2)
    c, _ = ops.grouped_moe_w8(x, gc, gs, dc, ds, 128, ids, (tw.float() * 2).to(torch.float16))
    assert torch.allclose(c.float(), 2 * a.float(), atol=2e-3, rtol=1e-2)
    z, _ = ops.grouped_moe_w8(x, gc, gs, dc, ds, 128, ids, torch.zeros(3, dtype=torch.float16))
    assert (z == 0).all()


# ---------------------------------------------------------------------------
# split-KV attention
# ---------------------------------------------------------------------------
def _qkv(ctx, seed, heads=4, d=64):
    g = _g(seed)
    return (torch.randn((heads, d), generator=g).to(torch.float16),
            torch.randn((heads, ctx, d), generator=g).to(torch.float16),
            torch.randn((heads, ctx, d), generator=g).to(torch.float16))


@pytest.mark.parametrize("filled", [1, 17, 300])
def test_split_kv_vs_dense_fp64(filled):
    q, k, v = _qkv(300, filled)
    out = ops.split_kv_oracle(q, k, v, filled, num_splits=5)
    ref = ops.dense_attention(q, k, v, filled)
    assert (out.double() - ref).abs().max() < 1e-5


def test_split_kv_count_invariance():
    q, k, v = _qkv(257, 1)
    outs = [ops.split_kv_oracle(q, k, v, 257, num_splits=s) for s in (1, 2, 3, 8, 17, 64)]
    for o in outs[1:]:
        assert (o - outs[0]).abs().max() < 1e-5


def test_split_kv_empty_and_nan_tail():
    q, k, v = _qkv(64, 2)
    assert (ops.split_kv_oracle(q, k, v, 0, num_splits=4) == 0).all()
    k2, v2 = k.clone(), v.clone()
    k2[:, 40:] = float("nan")
    v2[:, 40:] = float("nan")
    a = ops.split_kv_oracle(q, k, v, 40, num_splits=4)
    b = ops.split_kv_oracle(q, k2, v2, 40, num_splits=4)
    assert torch.isfinite(b).all() and torch.equal(a, b)


def test_int8_folded_vs_dequant_fp64_and_fold_identity():
    heads, ctx, d = 4, 200, 64
    q, k, v = _qkv(ctx, 3, heads, d)
    kc, ks = oq.kv_quantize_rows(k.numpy())
    vc, vs = oq.kv_quantize_rows(v.numpy())
    kc, ks, vc, vs = map(torch.from_numpy, (kc, ks, vc, vs))
    fold = ops.int8_attention_folded(q, kc, ks, vc, vs, ctx)
    deq = ops.int8_attention_dequant(q, kc, ks, vc, vs, ctx)
    assert (fold.double() - deq).abs().max() < 1e-3  # PARITY_GATE atol of the reference
    # the V scale multiplies the numerator only: dropping it from p*vs changes the answer
    wrong = ops.int8_attention_dequant(q, kc, ks, vc, torch.ones_like(vs), ctx)
    assert (wrong - deq).abs().max() > 1e-2
    # and the folded form agrees with the split-KV oracle on the dequantised cache
    kd = kc.float() * ks.float()[..., None]
    vd = vc.float() * vs.float()[..., None]
    ref = ops.split_kv_oracle(q, kd, vd, ctx, num_splits=3)
    assert (fold - ref).abs().max() < 1e-4


def test_dense_attention_single_token_is_v():
    q, k, v = _qkv(8, 4)
    out = ops.dense_attention(q, k, v, 1)
    assert torch.allclose(out, v[:, 0].double(), atol=0)
    scale = 1.0 / math.sqrt(64)
    s = (k[:, :3].double() @ q.double()[..., None])[..., 0] * scale
    w = torch.softmax(s, -1)
    assert torch.allclose(ops.dense_attention(q, k, v, 3), (w[..., None] * v[:, :3].double()).sum(1))
