"""torch-CPU restatements of the floating-point operators of the decode path.

Test infrastructure (see ``oracle/__init__.py``).  Each function names the
reference code it restates; the op order and rounding points follow it.
Inputs are CPU tensors.
"""

from __future__ import annotations

import math
from typing import Any

import numpy as np
import torch
import torch.nn.functional as F

LOG2E = 1.4426950408889634


# ---------------------------------------------------------------------------
# w8 dense GEMV
# ---------------------------------------------------------------------------
def dequant_w8(codes: Any, scale: Any, group: int) -> torch.Tensor:
    """``code * float(scale_fp16)`` per group, fp32 (``src/lemoq/kernels/reference.py:28-47``)."""
    c = codes.to(torch.float32)
    rows, cols = int(c.shape[0]), int(c.shape[1])
    s = scale.to(torch.float32).reshape(rows, cols // group, 1)
    return (c.reshape(rows, cols // group, group) * s).reshape(rows, cols)


def dequant_gemm_separate(x: Any, codes: Any, scale: Any, group: int, out_dtype: Any = None) -> torch.Tensor:
    """Materialise then GEMM: ``x.float() @ dequant(W).T`` (``src/lemoq/kernels/reference.py:50-60``).

    ``x`` may be narrower than the padded width (trailing weight columns unused).
    """
    w = dequant_w8(codes, scale, group)[:, : int(x.shape[-1])]
    y = x.to(torch.float32) @ w.t()
    return y.to(out_dtype) if out_dtype is not None else y


def dequant_weight_f16(codes: Any, scale: Any, group: int) -> torch.Tensor:
    """``QuantLinear.dequantized_weight(dtype=fp16)`` (``src/lemoq/quant/linear.py:365-395``):
    the exact fp32 product ``code * scale`` rounded once to fp16."""
    return dequant_w8(codes, scale, group).to(torch.float16)


def linear_separate_w8(x: Any, codes: Any, scale: Any, group: int) -> torch.Tensor:
    """The multi-token ``QuantLinear`` arm (``src/lemoq/quant/linear.py:471-480``):
    ``F.linear(x16, fp16 weight)`` -> fp16.  The product is formed in fp64 and
    rounded once to fp16 (a GPU fp32-accumulating GEMM lands within an ulp)."""
    w16 = dequant_weight_f16(codes, scale, group)[:, : int(x.shape[-1])]
    return (x.to(torch.float64) @ w16.to(torch.float64).t()).to(torch.float16)


def linear_f16(x: Any, weight: Any) -> torch.Tensor:
    """``F.linear`` of fp16 operands -> fp16 (fp64 product, one rounding)."""
    return (x.to(torch.float64) @ weight.to(torch.float64).t()).to(torch.float16)


def dequant_gemm_fused_tiles(x: Any, codes: Any, scale: Any, group: int, out_dtype: Any = None) -> torch.Tensor:
    """Group-by-group accumulation (``src/lemoq/kernels/reference.py:63-112``)."""
    M, K = int(x.shape[0]), int(x.shape[1])
    N, P = int(codes.shape[0]), int(codes.shape[1])
    xf = x.to(torch.float32)
    y = torch.zeros((M, N), dtype=torch.float32)
    for k0 in range(0, P, group):
        if k0 >= K:
            break
        hi = min(k0 + group, K)
        g = k0 // group
        w_tile = codes[:, k0:hi].to(torch.float32) * scale[:, g].to(torch.float32).unsqueeze(1)
        y += xf[:, k0:hi] @ w_tile.t()
    return y.to(out_dtype) if out_dtype is not None else y


# ---------------------------------------------------------------------------
# RMSNorm / RoPE
# ---------------------------------------------------------------------------
def rms_norm(x: Any, weight: Any, eps: float) -> torch.Tensor:
    """HF ``OlmoeRMSNorm.forward`` (transformers ``modeling_olmoe.py``; reference kernel contract
    ``src/lemoq/kernels/rmsnorm.py:184-202``): fp32 mean of squares, ``x*rsqrt`` rounded to the
    input dtype, then ``weight * that`` in the input dtype."""
    dt = x.dtype
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return weight * h.to(dt)


def clip_qkv(q: Any, k: Any, v: Any, clip: float | None):
    """HF OLMoE's ``clip_qkv`` (``OlmoeAttention.forward``; the reference's glue,
    ``src/lemoq/kernels/attn_decode.py:903-907``): ``clamp_(min=-clip, max=clip)``
    of the normed q, the normed k and v in their dtype, after q_norm/k_norm and
    before RoPE; ``None`` leaves them as they are."""
    if clip is None:
        return q, k, v
    c = float(clip)
    return q.clamp(min=-c, max=c), k.clamp(min=-c, max=c), v.clamp(min=-c, max=c)


def rotary_cos_sin(positions: Any, head_dim: int, theta: float = 10000.0):
    """HF ``OlmoeRotaryEmbedding`` (default rope): fp32 freqs, cos/sin cast to fp16."""
    pos = torch.as_tensor(positions, dtype=torch.int64).reshape(-1)
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = (inv_freq[None, :, None].float() @ pos[None, None, :].float()).transpose(1, 2)[0]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(torch.float16), emb.sin().to(torch.float16)


def rope_fused(x: Any, cos: Any, sin: Any) -> torch.Tensor:
    """``out = x*cos + sign*x[shift]*sin`` in fp32, rounded to x's dtype
    (``_rope_one_kernel``, ``src/lemoq/kernels/rope.py:101-123``).  x (..., D); cos/sin (D,)."""
    d = int(x.shape[-1])
    half = d // 2
    xf = x.to(torch.float32)
    shift = torch.cat((torch.arange(half, d), torch.arange(0, half)))
    sign = torch.cat((-torch.ones(half), torch.ones(d - half)))
    xs = xf[..., shift]
    y = xf * cos.to(torch.float32) + sign * xs * sin.to(torch.float32)
    return y.to(x.dtype)


def rope_hf(q: Any, k: Any, cos: Any, sin: Any) -> tuple[torch.Tensor, torch.Tensor]:
    """HF ``apply_rotary_pos_emb`` in the tensors' dtype (``rotate_half = cat(-x2, x1)``)."""

    def rotate_half(x: Any) -> Any:
        x1 = x[..., : x.shape[-1] // 2]
        x2 = x[..., x.shape[-1] // 2 :]
        return torch.cat((-x2, x1), dim=-1)

    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


# ---------------------------------------------------------------------------
# Routing and grouped MoE
# ---------------------------------------------------------------------------
def route(x: Any, router_weight: Any, top_k: int, norm_topk_prob: bool):
    """``moe_static._route`` (``src/lemoq/kernels/moe_static.py:262-283``): ``F.linear`` in x's
    dtype, fp32 softmax, top-k by probability (ties -> lowest index, the rule of
    ``_routing_triton.py:11-14``), optional renorm, weights cast to x's dtype."""
    logits = F.linear(x, router_weight)
    top_w, top_i = route_logits(logits, top_k, norm_topk_prob)
    return logits, top_w.to(x.dtype), top_i


def route_logits(logits: Any, top_k: int, norm_topk_prob: bool):
    """The softmax/top-k tail of ``_route`` on given logits: ``(top_w fp32, top_i int64)``."""
    p = F.softmax(logits, dim=-1, dtype=torch.float32)
    pn = p.numpy()
    order = np.argsort(-pn, axis=-1, kind="stable")[..., :top_k]
    top_i = torch.from_numpy(order.astype(np.int64))
    top_w = torch.gather(p, -1, top_i)
    if norm_topk_prob:
        top_w = top_w / top_w.sum(dim=-1, keepdim=True)
    return top_w, top_i


def grouped_gate_up_act(x: Any, gate_up_sel: Any, ffn: int) -> torch.Tensor:
    """``act[i] = silu(W_gate_i x) * (W_up_i x)`` in fp32 for the selected experts' fp32
    weights ``gate_up_sel`` (K, 2F, H) (``src/lemoq/kernels/moe_grouped.py:147-174``)."""
    xf = x.reshape(1, -1).to(torch.float32)
    xr = xf.repeat_interleave(int(gate_up_sel.shape[0]), dim=0)
    w = gate_up_sel.to(torch.float32)
    gate = (w[:, :ffn, :] @ xr.unsqueeze(-1)).squeeze(-1)
    up = (w[:, ffn:, :] @ xr.unsqueeze(-1)).squeeze(-1)
    return gate * torch.sigmoid(gate) * up


def grouped_down_sum(act: Any, down_sel: Any, top_w: Any) -> torch.Tensor:
    """``out = sum_i top_w_i * (W_down_i act_i)`` in fp32 (``src/lemoq/kernels/moe_grouped.py:177-195``)."""
    af = act.to(torch.float32)
    w = down_sel.to(torch.float32)
    y = torch.matmul(w, af.unsqueeze(-1)).squeeze(-1)
    y = y * top_w.reshape(-1, 1).to(torch.float32)
    return y.sum(dim=0)


def grouped_moe_w8(x: Any, gu_codes: Any, gu_scale: Any, dn_codes: Any, dn_scale: Any, group: int,
                   ids: Any, top_w: Any) -> tuple[torch.Tensor, torch.Tensor]:
    """``grouped_moe_forward_quant`` numerics (``src/lemoq/kernels/moe_grouped_quant.py:473-523``):
    dequantise the selected experts, act rounded to fp16, down + weighted sum in fp32, fp16 out.
    Returns ``(out fp16 (H,), act fp16 (K, F))``."""
    ids = [int(i) for i in ids.reshape(-1).tolist()]
    ffn = int(gu_codes.shape[1]) // 2
    gu = torch.stack([dequant_w8(gu_codes[e], gu_scale[e], group) for e in ids])
    act = grouped_gate_up_act(x, gu, ffn).to(torch.float16)
    dn = torch.stack([dequant_w8(dn_codes[e], dn_scale[e], group) for e in ids])
    out = grouped_down_sum(act, dn, top_w.reshape(-1).to(torch.float16)).to(torch.float16)
    return out, act


def moe_prefill_w8(x: Any, gu_codes: Any, gu_scale: Any, dn_codes: Any, dn_scale: Any, group: int,
                   top_i: Any, top_w16: Any) -> torch.Tensor:
    """``_prefill_forward`` with quantized experts (``src/lemoq/kernels/moe_static.py:329-371``):
    experts in ascending order; the expert's tokens (``nonzero``, token order) go through
    ``gu = F.linear(x_e, fp16 W_gu)``, ``act = silu(gate) * up`` and ``y = F.linear(act, fp16 W_dn)``
    in fp16, and ``y * w`` is index_added into a zero fp16 output.  x (T, H) fp16;
    top_i (T, k) int64; top_w16 (T, k) fp16 -> (T, H) fp16."""
    out = torch.zeros_like(x)
    ffn = int(gu_codes.shape[1]) // 2
    for e in range(int(gu_codes.shape[0])):
        tok, slot = (top_i == e).nonzero(as_tuple=True)
        if tok.numel() == 0:
            continue
        w = top_w16[tok, slot].unsqueeze(-1)
        gu = linear_separate_w8(x[tok], gu_codes[e], gu_scale[e], group)
        act = F.silu(gu[:, :ffn]) * gu[:, ffn:]
        y = linear_separate_w8(act, dn_codes[e], dn_scale[e], group)
        out.index_add_(0, tok, y * w)
    return out


def causal_attention(q: Any, k: Any, v: Any, *, scale: float | None = None,
                     dtype: Any = torch.float64) -> torch.Tensor:
    """Causal softmax attention over the prompt (HF ``OlmoeAttention`` with sdpa and a causal
    mask), in fp64 by default.  q, k, v (T, H, D) -> (T, H, D)."""
    T, dim = int(q.shape[0]), int(q.shape[-1])
    scale = (1.0 / math.sqrt(dim)) if scale is None else float(scale)
    qq, kk, vv = (t.to(dtype).transpose(0, 1) for t in (q, k, v))
    scores = torch.matmul(qq, kk.transpose(1, 2)) * scale
    future = torch.ones((T, T), dtype=torch.bool).triu(1)
    scores = scores.masked_fill(future, float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), vv).transpose(0, 1)


# ---------------------------------------------------------------------------
# Split-KV attention (fp16) and its oracles
# ---------------------------------------------------------------------------
def split_kv_partials(q: Any, k: Any, v: Any, filled: int, *, num_splits: int, scale: float | None = None,
                      block_n: int = 128):
    """Per-split online-softmax partials in the kernel's block order
    (``split_kv_partials_reference``, ``src/lemoq/kernels/attn_decode.py:295-354``).
    q (H, D); k, v (H, S, D) -> m, l (H, NS) and acc (H, NS, D), fp32."""
    qf, kf, vf = q.to(torch.float32), k.to(torch.float32), v.to(torch.float32)
    heads, dim = int(qf.shape[0]), int(qf.shape[1])
    scale = (1.0 / math.sqrt(dim)) if scale is None else float(scale)
    qk_scale = scale * LOG2E
    m = torch.full((heads, num_splits), float("-inf"))
    l = torch.zeros((heads, num_splits))
    acc = torch.zeros((heads, num_splits, dim))
    n = int(filled)
    if n == 0:
        return m, l, acc
    chunk = -(-n // num_splits)
    for s in range(num_splits):
        start, end = s * chunk, min(s * chunk + chunk, n)
        if start >= end:
            continue
        m_i = torch.full((heads,), float("-inf"))
        l_i = torch.zeros((heads,))
        a_i = torch.zeros((heads, dim))
        for n0 in range(start, end, block_n):
            hi = min(n0 + block_n, end)
            qk = torch.matmul(kf[:, n0:hi, :], qf.unsqueeze(-1)).squeeze(-1) * qk_scale
            m_new = torch.maximum(m_i, qk.max(dim=1).values)
            alpha = torch.exp2(m_i - m_new)
            p = torch.exp2(qk - m_new.unsqueeze(1))
            l_i = l_i * alpha + p.sum(dim=1)
            a_i = a_i * alpha.unsqueeze(1) + torch.matmul(p.unsqueeze(1), vf[:, n0:hi, :]).squeeze(1)
            m_i = m_new
        m[:, s], l[:, s], acc[:, s] = m_i, l_i, a_i
    return m, l, acc


def merge_splits(m: Any, l: Any, acc: Any) -> torch.Tensor:
    """LSE merge (``merge_splits_reference``, ``src/lemoq/kernels/attn_decode.py:357-379``)."""
    big_m = m.max(dim=1, keepdim=True).values
    big_m = torch.where(torch.isfinite(big_m), big_m, torch.zeros_like(big_m))
    w = torch.exp2(m - big_m)
    num = (acc * w.unsqueeze(-1)).sum(dim=1)
    den = (l * w).sum(dim=1)
    safe = den.clamp_min(torch.finfo(torch.float32).tiny).unsqueeze(1)
    return torch.where(den.unsqueeze(1) > 0, num / safe, num)


def split_kv_oracle(q: Any, k: Any, v: Any, filled: int, *, num_splits: int, scale: float | None = None) -> torch.Tensor:
    return merge_splits(*split_kv_partials(q, k, v, filled, num_splits=num_splits, scale=scale))


def dense_attention(q: Any, k: Any, v: Any, filled: int, *, scale: float | None = None,
                    dtype: Any = torch.float64) -> torch.Tensor:
    """Unsplit softmax attention, fp64 by default (``dense_attention_oracle``,
    ``src/lemoq/kernels/attn_decode.py:400-423``).  q (H, D); k, v (H, S, D)."""
    heads, dim = int(q.shape[0]), int(q.shape[1])
    n = int(filled)
    if n == 0:
        return torch.zeros((heads, dim), dtype=dtype)
    scale = (1.0 / math.sqrt(dim)) if scale is None else float(scale)
    qq = q.to(dtype)
    kk = k[:, :n, :].to(dtype)
    vv = v[:, :n, :].to(dtype)
    scores = torch.matmul(kk, qq.unsqueeze(-1)).squeeze(-1) * scale
    w = torch.softmax(scores, dim=-1)
    return torch.matmul(w.unsqueeze(1), vv).squeeze(1)


def int8_attention_folded(q: Any, kc: Any, ks: Any, vc: Any, vs: Any, filled: int, *,
                          scale: float | None = None) -> torch.Tensor:
    """KV-INT8 attention with the reference's fold algebra (``_attn_split_kernel_int8``,
    ``src/lemoq/kernels/_attn_triton.py:143-161``) as one split, fp32:
    ``s_t = ((q.c_t)*QK_SCALE)*ks_t``, ``p = exp2(s - max)``, ``out = sum (p*vs)*c / sum p``.
    q (H, D) fp16; kc, vc (H, S, D) int8; ks, vs (H, S) fp16 -> (H, D) fp32."""
    heads, dim = int(q.shape[0]), int(q.shape[1])
    n = int(filled)
    if n == 0:
        return torch.zeros((heads, dim))
    scale = (1.0 / math.sqrt(dim)) if scale is None else float(scale)
    qk_scale = scale * LOG2E
    qf = q.to(torch.float32)
    c = kc[:, :n, :].to(torch.float32)
    s = (torch.matmul(c, qf.unsqueeze(-1)).squeeze(-1) * qk_scale) * ks[:, :n].to(torch.float32)
    m = s.max(dim=1, keepdim=True).values
    p = torch.exp2(s - m)
    pw = p * vs[:, :n].to(torch.float32)
    num = torch.matmul(pw.unsqueeze(1), vc[:, :n, :].to(torch.float32)).squeeze(1)
    return num / p.sum(dim=1, keepdim=True)


def int8_attention_dequant(q: Any, kc: Any, ks: Any, vc: Any, vs: Any, filled: int, *,
                           scale: float | None = None, dtype: Any = torch.float64) -> torch.Tensor:
    """Dequantise-then-attend oracle (``tests/test_kv_int8_read_gpu.py:69-87`` of the reference):
    ``k = c*s``, ``v = c*s``, then dense attention in fp64."""
    k = kc.to(dtype) * ks.to(dtype).unsqueeze(-1)
    v = vc.to(dtype) * vs.to(dtype).unsqueeze(-1)
    return dense_attention(q, k, v, filled, scale=scale, dtype=dtype)


def write_kv_slot(keys: Any, values: Any, pos: int, k_new: Any, v_new: Any) -> None:
    """Slot write contract (``write_kv_slot``, ``src/lemoq/kernels/kv_write.py:26-50``):
    keys/values (1,H,S,D) in place, only ``[pos : pos+q_len]`` changes."""
    q_len = int(k_new.shape[2])
    keys[:, :, pos : pos + q_len, :] = k_new
    values[:, :, pos : pos + q_len, :] = v_new
