"""CPU checks of the C-ABI library: it loads without a GPU and exports every
symbol include/lemoq_hip.h declares, with the status strings of the header."""

from __future__ import annotations

import ctypes
import math
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "lemoq_hip.h")


def _declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lemoq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    names = _declared_functions()
    assert "lemoq_olmoe_decode_step" in names and "lemoq_gemv_w8" in names
    assert len(names) >= 19


def test_library_exports_every_declared_symbol():
    from lemoq import _hip

    if not _hip.library_available():
        pytest.fail("liblemoq_hip.so is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(_hip.LIB_PATH)
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # every declared function has a typed ctypes signature
    assert sorted(_hip.SIGNATURES) == _declared_functions()


def test_status_strings_and_abi():
    from lemoq import _hip

    lib = _hip.load()
    assert lib.lemoq_abi_version() == _hip.ABI_VERSION
    assert lib.lemoq_status_string(0) == b"ok"
    assert b"NULL" in lib.lemoq_status_string(-1)
    assert b"unknown" in lib.lemoq_status_string(-99)


def test_argument_rejection_happens_before_any_launch():
    """Invalid arguments return a negative status without touching a device."""
    from lemoq import _hip

    lib = _hip.load()
    assert lib.lemoq_gemv_w8(None, 1, 16, None, None, 16, 16, 16, None, 1, None) == -1
    # aligned non-null fake pointers, bad group (not a multiple of 16): rejected as unsupported
    fake = 4096
    assert lib.lemoq_gemv_w8(fake, 1, 128, fake, fake, 8, 128, 8, fake, 1, None) == -3
    assert lib.lemoq_gemv_w8(fake, 1, 128, fake + 1, fake, 8, 128, 128, fake, 1, None) == -4
    assert lib.lemoq_attn_split_i8(fake, fake, fake, fake, fake, 128 * 10, 10, fake, 16, 96, 4, 1.0,
                                   fake, fake, fake, None) == -3
    assert lib.lemoq_route_topk(fake, 1, 1, 2000, 2000, 8, 0, fake, fake, None) == -2
    # prefill GEMMs: K not a multiple of 32, group not a multiple of 32, misaligned codes
    assert lib.lemoq_gemm_w8(fake, 4, 48, 48, None, fake, fake, 64, 48, fake, 64, None, 0, None) == -2
    assert lib.lemoq_gemm_w8(fake, 4, 128, 128, None, fake, fake, 64, 16, fake, 64, None, 0, None) == -3
    assert lib.lemoq_gemm_w8(fake, 4, 128, 128, None, fake + 8, fake, 64, 128, fake, 64, None, 0, None) == -4
    assert lib.lemoq_gemm_f16(fake, 4, 128, 64, fake, 64, fake, 64, None) == -2
    # split-K: K not a multiple of 64 * splits, a missing workspace, too many splits
    assert lib.lemoq_gemm_f16_splitk(fake, 4, 192, 192, fake, 64, fake, 64, 2, fake, None) == -2
    assert lib.lemoq_gemm_f16_splitk(fake, 4, 256, 256, fake, 64, fake, 64, 2, None, None) == -1
    assert lib.lemoq_gemm_f16_splitk(fake, 4, 256, 256, fake, 64, fake, 64, 65, fake, None) == -2
    # partials only (y NULL) needs splits > 1; the routing of partials bounds splits and E
    assert lib.lemoq_gemm_f16_splitk(fake, 4, 256, 256, fake, 64, None, 64, 1, fake, None) == -1
    assert lib.lemoq_route_topk_splitk(fake, 65, 4, 64, 8, 0, fake, fake, None) == -2
    assert lib.lemoq_route_topk_splitk(fake, 0, 4, 64, 8, 0, fake, fake, None) == -2
    assert lib.lemoq_route_topk_splitk(fake, 4, 4, 2000, 8, 0, fake, fake, None) == -2
    assert lib.lemoq_route_topk_splitk(None, 4, 4, 64, 8, 0, fake, fake, None) == -1
    # prefill entry points
    assert lib.lemoq_gather_rows(fake, 10, 12, fake, 3, fake, None) == -2            # H % 8
    assert lib.lemoq_gather_rows(fake, 10, 16, fake, 3, fake + 8, None) == -4        # dst alignment
    assert lib.lemoq_attn_prefill_f16(fake, 256, fake, fake, 256 * 8, 8, 2, 96, 1.0, fake, 256, None) == -3
    assert lib.lemoq_attn_prefill_f16(fake, 256, fake, fake, 128 * 4, 8, 2, 128, 1.0, fake, 256, None) == -2
    assert lib.lemoq_qk_norm_rope_kv_i8_rows(fake, 10, 2, 128, fake, fake, 1e-5, fake, fake, 5, fake, fake, fake,
                                             fake, fake, 16 * 128, 12, None, None, 0, math.inf, None) == -2  # rows past s_len
    for bad in (-1.0, math.nan):  # clip_qkv must be >= 0 (+inf disables it)
        assert lib.lemoq_qk_norm_rope_kv_i8_rows(fake, 10, 2, 128, fake, fake, 1e-5, fake, fake, 0, fake, fake,
                                                 fake, fake, fake, 16 * 128, 12, None, None, 0, bad, None) == -2
        assert lib.lemoq_qk_norm_rope_kv_i8(fake, 2, 128, fake, fake, 1e-5, fake, fake, fake, fake, fake, fake,
                                            fake, fake, 16 * 128, 12, None, None, 0, None, bad, None) == -2
        assert lib.lemoq_attn_split_fused_i8(fake, 16, 128, fake, fake, 1e-5, fake, fake, fake, fake, fake, fake,
                                             fake, 1100 * 128, 1100, 16, 0.1, fake, fake, fake, bad, None) == -2
        assert lib.lemoq_attn_split_fused_f16(fake, 16, 128, fake, fake, 1e-5, fake, fake, fake, fake, fake,
                                              1100 * 128, 1100, 16, 0.1, fake, fake, fake, bad, None) == -2
    f16 = lambda *a: lib.lemoq_attn_split_fused_f16(fake, *a)  # noqa: E731
    assert f16(16, 128, fake, fake, 1e-5, fake, fake, fake, None, fake, 1100 * 128, 1100, 16, 0.1, fake, fake,
               fake, math.inf, None) == -1                                          # no k cache
    assert f16(16, 96, fake, fake, 1e-5, fake, fake, fake, fake, fake, 1100 * 96, 1100, 16, 0.1, fake, fake,
               fake, math.inf, None) == -3                                          # head_dim
    assert f16(16, 128, fake, fake, 1e-5, fake, fake, fake, fake, fake, 1000 * 128, 1100, 16, 0.1, fake, fake,
               fake, math.inf, None) == -2                                          # head stride < s_len * D
    assert f16(16, 128, fake, fake, 1e-5, fake, fake, fake, fake + 2, fake, 1100 * 128, 1100, 16, 0.1, fake, fake,
               fake, math.inf, None) == -4                                          # k cache alignment
    assert f16(16, 128, fake, fake, 1e-5, fake, fake, fake, fake, fake, 1100 * 128 + 4, 1100, 16, 0.1, fake,
               fake, fake, math.inf, None) == -4                                    # rows 16-byte aligned
    # the prefill rows: all four KV-INT8 buffers, or none of them and both fp16 caches
    rows = lambda kc, ks, kf, vf: lib.lemoq_qk_norm_rope_kv_i8_rows(  # noqa: E731
        fake, 10, 2, 128, fake, fake, 1e-5, fake, fake, 20, fake, kc, ks, fake, fake, 16 * 128, 12, kf, vf,
        16 * 128, math.inf, None)
    assert rows(fake, None, None, None) == -1                                       # half the KV-INT8 buffers
    assert lib.lemoq_qk_norm_rope_kv_i8_rows(fake, 10, 2, 128, fake, fake, 1e-5, fake, fake, 20, fake, None,
                                             None, None, None, 16 * 128, 12, fake, None, 16 * 128, math.inf,
                                             None) == -1                            # fp16 only: v cache missing
    assert lib.lemoq_qk_norm_rope_kv_i8_rows(fake, 10, 2, 128, fake, fake, 1e-5, fake, fake, 20, fake, None,
                                             None, None, None, 0, 12, fake, fake, 16 * 128, math.inf,
                                             None) == -2                            # fp16 only: rows past s_len
    assert lib.lemoq_moe_prefill_max_tiles(8192, 64) == 8192 // 128 + 64
    assert lib.lemoq_moe_prefill_sort(fake, fake, 4097, 8, 64, fake, fake, fake, fake, fake, 10 ** 6, None) == -3
    assert lib.lemoq_moe_prefill_sort(fake, fake, 16, 8, 300, fake, fake, fake, fake, fake, 10 ** 6, None) == -2
    assert lib.lemoq_moe_prefill_sort(fake, fake, 16, 8, 64, fake, fake, fake, fake, fake, 10, None) == -2
    assert lib.lemoq_moe_prefill_gate_up(fake, 2048, fake, fake, 64, fake, fake, 1000, 128, fake, None) == -2
    assert lib.lemoq_moe_prefill_down(fake, 1024, fake, fake, fake, 64, fake + 4, fake, 2048, 128, fake, None) == -4
    assert lib.lemoq_moe_prefill_combine(fake, fake, 4, 9, 2048, None, fake, None) == -2
    # combine + next norm: H past the LDS row, xn overlapping out, a missing norm weight
    cn = lambda T, H, out, w, xn: lib.lemoq_moe_prefill_combine_norm(  # noqa: E731
        1 << 24, fake, T, 8, H, None, out, w, 1e-5, xn, None)
    assert cn(4, 8200, 1 << 20, fake, 1 << 22) == -2
    assert cn(4, 2048, 1 << 20, fake, (1 << 20) + 4096) == -2
    assert cn(4, 2048, 1 << 20, None, 1 << 22) == -1
    assert cn(4, 2048, 1 << 20, fake + 2, 1 << 22) == -4      # norm weight misaligned
    assert cn(4, 2048, 1 << 20, fake, (1 << 22) + 8) == -4    # xn_out misaligned
    # fused merge + o_proj: head_dim 64 and 6 heads unsupported, N % 32, too many splits, misaligned codes
    assert lib.lemoq_attn_merge_o_proj_w8(fake, fake, fake, 16, 16, 64, fake, fake, 2048, 128, fake, None) == -3
    assert lib.lemoq_attn_merge_o_proj_w8(fake, fake, fake, 6, 16, 128, fake, fake, 2048, 128, fake, None) == -3
    assert lib.lemoq_attn_merge_o_proj_w8(fake, fake, fake, 16, 16, 128, fake, fake, 2040, 128, fake, None) == -2
    assert lib.lemoq_attn_merge_o_proj_w8(fake, fake, fake, 16, 65, 128, fake, fake, 2048, 128, fake, None) == -2
    assert lib.lemoq_attn_merge_o_proj_w8(fake, fake, fake, 16, 16, 128, fake + 4, fake, 2048, 128, fake, None) == -4
    assert lib.lemoq_attn_merge_o_proj_w8(None, fake, fake, 16, 16, 128, fake, fake, 2048, 128, fake, None) == -1
    # router after the partials: hidden 1024 and 3 partial rows unsupported, h_out overlapping h
    rr = lambda part, npart, h, hidden, h_out: lib.lemoq_router_logits_resid(  # noqa: E731
        part, npart, h, fake, 1e-5, hidden, fake, 64, h_out, fake, fake, None)
    assert rr(fake, 4, 1 << 20, 1024, 1 << 21) == -3
    assert rr(fake, 3, 1 << 20, 2048, 1 << 21) == -3
    assert rr(fake, 4, 1 << 20, 2048, (1 << 20) + 2048) == -2
    assert rr(fake + 4, 4, 1 << 20, 2048, 1 << 21) == -4
    assert rr(fake, 4, 1 << 20, 2048, None) == -1
    # weight formats: unknown format, MXFP4 with fp32 scales / group 64 / a zero point, missing zero point,
    # group not a multiple of the 16-byte slice, padded_k past 8192, misaligned codes, K > padded_k
    gq = lambda fmt, zero, s32, pk, g, codes=fake, M=1, K=128: lib.lemoq_gemv_q(  # noqa: E731
        fake, M, K, codes, fmt, fake, zero, s32, 64, pk, g, fake, 1, None)
    assert gq(5, None, 0, 128, 128) == -3
    assert gq(4, None, 1, 128, 32) == -3 and gq(4, None, 0, 128, 64) == -3 and gq(4, fake, 0, 128, 32) == -3
    assert gq(1, None, 0, 128, 128) == -1 and gq(3, None, 0, 128, 128) == -1
    assert gq(2, None, 0, 128, 16) == -3 and gq(0, None, 0, 128, 8) == -3
    assert gq(2, None, 0, 16384, 128) == -3
    assert gq(2, None, 0, 128, 128, codes=fake + 8) == -4
    assert gq(0, None, 0, 128, 128, K=256) == -2 and gq(0, None, 0, 128, 128, M=0) == -2
    assert gq(4, None, 0, 128, 32, M=70000) == -2
    assert lib.lemoq_dequant_q(fake, 2, fake, None, 0, 64, 128, 128, fake, 100, 129, 0, None) == -2  # k_out > padded
    assert lib.lemoq_dequant_q(fake, 2, fake, None, 0, 64, 128, 128, fake, 100, 120, 0, None) == -2  # ld < k_out
    assert lib.lemoq_rtn_quantize(fake, 4, 130, 7, 4, 1, fake, None, None, None, None, None) == -2   # odd group at 4 bits
    assert lib.lemoq_rtn_quantize(fake, 4, 130, 128, 6, 1, fake, None, None, None, None, None) == -3
    assert lib.lemoq_mxfp4_quantize(fake, 4, 0, fake, fake, None) == -2
    assert lib.lemoq_fake_quant_rows(fake, 4, 0, fake, None) == -2
    # o_proj + residual of the 4-bit step: residual required; y itself or apart from it
    gr = lambda res, y, M=1, N=64: lib.lemoq_gemv_q_residual(  # noqa: E731
        fake, M, 128, fake, 2, fake, None, 0, N, 128, 128, res, y, None)
    assert gr(None, 1 << 22) == -1 and gr(1 << 22, None) == -1
    assert gr(1 << 22, (1 << 22) + 64) == -2                # partial overlap
    assert gr(1 << 22, 1 << 23, N=64, M=0) == -2            # then the GEMV's own rules
    # 4-bit q|k|v GEMV with the input norm: norm weight required, eps >= 0, fp16 scales only
    gn = lambda nw=fake, eps=1e-5, s32=0, idx=None, M=1, K=128, copy=None: lib.lemoq_gemv_q_rmsnorm(  # noqa: E731
        fake, idx, 10, M, K, nw, eps, copy, fake, 2, fake, None, s32, 64, K, 128, fake, 1, None)
    assert gn(nw=None) == -1 and gn(eps=-1.0) == -2 and gn(eps=math.nan) == -2 and gn(s32=1) == -3
    assert gn(idx=fake, M=2) == -2                           # a gathered row is one row
    assert gn(copy=fake) == -3                               # x_copy needs the per-block form (K 128: per wave)
    # routed 4-bit gate/up: ids/weights outputs, top_k <= min(64, E), E <= 256, 4-bit groups
    gu = lambda E=64, K=8, g=128, ti=fake, tw=fake: lib.lemoq_moe_gate_up_w4_routed(  # noqa: E731
        fake, fake, fake, fake, K, 0, E, 1024, 2048, g, fake, ti, tw, None)
    assert gu(ti=None) == -1 and gu(tw=None) == -1
    assert gu(K=65, E=128) == -2 and gu(E=4, K=8) == -2
    assert gu(E=300) == -3 and gu(g=16) == -3
    with pytest.raises(ValueError):
        _hip.call("lemoq_gemv_w8", None, 1, 16, None, None, 16, 16, 16, None, 1, None)


def _fake_step(**over):
    """A LemoqOlmoeStep at the OLMoE shape whose pointers are aligned fakes (never
    dereferenced: these cases are rejected before anything is launched)."""
    from lemoq import _hip

    layers = (_hip.LemoqOlmoeLayer * 2)()
    addr = [1 << 24]

    def nxt():
        addr[0] += 1 << 16
        return addr[0]

    for L in layers:
        for name, _ in _hip.LemoqOlmoeLayer._fields_:
            setattr(L, name, nxt())
    st = _hip.LemoqOlmoeStep()
    shape = dict(hidden=2048, heads=16, head_dim=128, ffn=1024, num_experts=64, top_k=8, vocab=50304, group=128,
                 num_layers=2, max_seq=1100, num_splits=16, norm_topk_prob=0)
    for k, v in shape.items():
        setattr(st, k, v)
    st.eps, st.qk_scale, st.clip_qkv = 1e-5, 0.1, math.inf
    st.layers = ctypes.cast(layers, ctypes.POINTER(_hip.LemoqOlmoeLayer))
    for name, typ in _hip.LemoqOlmoeStep._fields_:
        if typ is ctypes.c_void_p:
            setattr(st, name, nxt())
    st.prompt_len, st.history_len = 4, 1200
    st.am_len = int(_hip.load().lemoq_lm_head_argmax_parts(50304))
    st.weight_bits, st.lm_f16 = 8, None  # the w8a16 cell with the W8 lm_head
    for k, v in over.items():
        setattr(st, k, v)
    return st, layers


def test_decode_step_rejects_before_any_launch():
    """Every rule of every launch of the step is checked before the first launch
    (so a rejected step leaves the KV cache and buffers untouched).  Each case
    below would otherwise be rejected by a launch in the middle of the step
    (the routed gate/up, the down projection, the lm_head argmax, the merge);
    a negative status proves nothing was enqueued: on this GPU-less host a
    launch attempt would return a positive HIP error instead."""
    from lemoq import _hip

    lib = _hip.load()
    step = lambda **over: lib.lemoq_olmoe_decode_step(ctypes.byref(_fake_step(**over)[0]), None)  # noqa: E731
    parts = int(lib.lemoq_lm_head_argmax_parts(50304))
    assert step(am_len=parts - 1) == -2                    # lm_head argmax partials (last launch)
    assert step(num_experts=300) == -3                      # routed gate/up: > 256 experts
    assert step(top_k=65) == -2                             # gate/up / down: top_k > 64
    assert step(ffn=1000) == -3                             # down: ffn % 16
    assert step(group=8) == -3                              # every GEMV: group % 16
    assert step(head_dim=96) == -3                          # attention: head_dim
    assert step(act=(1 << 30) + 8) == -4                    # down: act alignment
    assert step(clip_qkv=-1.0) == -2 and step(clip_qkv=math.nan) == -2  # attention: clip_qkv bound
    st, layers = _fake_step()
    layers[1].dn_codes = (1 << 30) + 4                      # layer 1's down codes misaligned
    assert lib.lemoq_olmoe_decode_step(ctypes.byref(st), None) == -4
    st, layers = _fake_step()
    layers[1].router = None                                 # layer 1's router missing
    assert lib.lemoq_olmoe_decode_step(ctypes.byref(st), None) == -1
    # unfused attention-output path (no o_part): merge split bound
    assert step(o_part=None, num_splits=2000) == -2
    # cache kind: 0 or 1 only; the fp16 cache needs no scales, KV-INT8 does
    assert step(kv_fp16=2) == -2
    st, layers = _fake_step(kv_fp16=1)
    layers[0].ks = layers[0].vs = None                      # no scales: fine for fp16 rows,
    st.h_mid = st.h                                         # so the rule after the layers rejects
    assert lib.lemoq_olmoe_decode_step(ctypes.byref(st), None) == -2
    st, layers = _fake_step()
    layers[0].ks = None                                     # KV-INT8 without its scales
    assert lib.lemoq_olmoe_decode_step(ctypes.byref(st), None) == -1
    # weight bits 8 or 4; the 4-bit layer's GEMV / MoE rules; the fp16 lm_head's
    assert step(weight_bits=0) == -3 and step(weight_bits=5) == -3
    assert step(weight_bits=4, group=16) == -3              # 4-bit groups of 32
    assert step(weight_bits=4, ffn=1008) == -3              # 4-bit down: ffn % 32
    assert step(weight_bits=4, num_splits=2000) == -2       # the merge of the 4-bit layer
    assert step(weight_bits=4, attn=(1 << 30) + 8) == -4    # merge output / o_proj input alignment
    assert step(weight_bits=4, num_experts=300) == -3       # routed 4-bit gate/up: > 256 experts
    big = 1 << 30
    assert step(lm_f16=big, am_len=parts - 1) == -2         # the fp16 lm_head writes the same partials
    assert step(lm_f16=big, am_val=None) == -1
    assert step(lm_f16=big + 8) == -4                       # fp16 lm_head alignment
    # with an fp16 lm_head the W8 lm_head may be absent (a later rule rejects)
    assert step(lm_f16=big, lm_codes=None, lm_scale=None, top_k=65) == -2
    assert step(lm_codes=None) == -1 and step(am_idx=None) == -1
