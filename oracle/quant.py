"""numpy restatements of the bit-exact quantisers and of the routing order.

Test infrastructure (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import math
from typing import Any

import numpy as np


def rtn_quantize_w8(weight: Any, group_size: int = 128) -> dict[str, Any]:
    """Symmetric per-group RTN, 8-bit.

    Restates ``quantize_rtn`` of ``src/lemoq/quant/numpy_oracle.py:58-116`` for
    ``bits=8, symmetric=True``: pad the input dim to a multiple of the group
    with zeros, ``scale = absmax/127`` in fp32 (1.0 when absmax == 0),
    ``codes = clip(round_half_even(w/scale), -128, 127)``.  Adds the fp16 cast
    of the scale stored by the packed formats
    (``src/lemoq/kernels/moe_grouped_quant.py:232``, ``src/lemoq/quant/linear.py:332``).
    """
    w = np.asarray(weight, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError("2-D weights only")
    out_f, in_f = w.shape
    n_groups = int(math.ceil(in_f / group_size))
    padded_in = n_groups * group_size
    if padded_in != in_f:
        pad = np.zeros((out_f, padded_in), dtype=np.float32)
        pad[:, :in_f] = w
        w = pad
    grouped = w.reshape(out_f, n_groups, group_size)
    absmax = np.max(np.abs(grouped), axis=2, keepdims=True)
    scale = np.where(absmax > 0, absmax / np.float32(127), np.float32(1.0)).astype(np.float32)
    codes = np.clip(np.round(grouped / scale), -128, 127).astype(np.int8)
    scale2 = scale.reshape(out_f, n_groups)
    return {
        "codes_padded": codes.reshape(out_f, padded_in),
        "scale": scale2,
        "scale_f16": scale2.astype(np.float16),
        "n_groups": n_groups,
        "padded_in": padded_in,
        "shape": (out_f, in_f),
    }


def rtn_dequant(codes: Any, scale: Any, group_size: int) -> np.ndarray:
    """``code * float(scale)`` per group, fp32 (``src/lemoq/quant/linear.py:365-395``,
    ``src/lemoq/kernels/moe_grouped_quant.py:145-157``)."""
    c = np.asarray(codes).astype(np.float32)
    s = np.asarray(scale).astype(np.float32)
    rows, cols = c.shape
    return (c.reshape(rows, cols // group_size, group_size) * s[:, :, None]).reshape(rows, cols)


def kv_quantize_rows(x: Any) -> tuple[np.ndarray, np.ndarray]:
    """Per-token symmetric int8 along the last axis.

    Restates ``quantize_per_token_int8`` (``src/lemoq/kernels/kv_int8.py:30-41``):
    fp32 amax, ``s = amax/127`` (1.0 when amax == 0), ``q = round_half_even(x/s)``
    clamped to [-127, 127], scale returned as fp16.
    """
    xf = np.asarray(x).astype(np.float32)
    amax = np.max(np.abs(xf), axis=-1, keepdims=True)
    s = np.where(amax > 0, amax / np.float32(127), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.round(xf / s), -127, 127).astype(np.int8)
    return q, s[..., 0].astype(np.float16)


def route_order(logits: Any, top_k: int, norm: bool) -> tuple[np.ndarray, np.ndarray]:
    """fp32 softmax -> top-k by a stable descending sort (ties -> lowest index) -> optional renorm.

    Restates the reference's numpy routing oracle (``tests/test_routing_fusion.py:24-35``)
    with the tie rule of ``_routing_triton.py:11-14``.
    """
    z = np.asarray(logits).astype(np.float32)
    z = z - z.max(axis=-1, keepdims=True)
    e = np.exp(z)
    w = e / e.sum(axis=-1, keepdims=True)
    order = np.argsort(-w, axis=-1, kind="stable")
    idx = order[..., :top_k]
    top_w = np.take_along_axis(w, idx, axis=-1)
    if norm:
        top_w = top_w / top_w.sum(axis=-1, keepdims=True)
    return top_w.astype(np.float32), idx.astype(np.int64)


def rtn_quantize(weight: Any, bits: int = 4, group_size: int = 128, symmetric: bool = True) -> dict[str, Any]:
    """Per-group RTN at 4 or 8 bits, symmetric or asymmetric.

    Restates ``quantize_rtn`` of ``src/lemoq/quant/numpy_oracle.py:58-107``
    (the torch twin ``src/lemoq/quant/rtn.py:38-99`` is bit-identical to it,
    ``tests/test_quant_oracle.py:104-117``): zero-pad the input dim to the
    group; symmetric ``scale = absmax/qmax`` (1 when 0), ``codes =
    clip(round(w/scale), -qmax-1, qmax)``; asymmetric over the real columns
    only, ``scale = (max-min)/qmax`` (1 when 0), ``zero = round(-min/scale)``,
    ``codes = clip(round(w/scale) + zero, 0, qmax)``.  fp32, round half to even.
    Codes are returned as int32 like the reference, plus the fp16 casts of
    scale and zero that ``QuantLinear`` stores (``src/lemoq/quant/linear.py:330-340``).
    """
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    w = np.asarray(weight, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError("2-D weights only")
    out_f, in_f = w.shape
    n_groups = int(math.ceil(in_f / group_size))
    padded_in = n_groups * group_size
    if padded_in != in_f:
        pad = np.zeros((out_f, padded_in), dtype=np.float32)
        pad[:, :in_f] = w
        w = pad
    grouped = w.reshape(out_f, n_groups, group_size)
    qmax = (2 ** (bits - 1)) - 1 if symmetric else (2 ** bits) - 1
    if symmetric:
        absmax = np.max(np.abs(grouped), axis=2, keepdims=True)
        scale = np.where(absmax > 0, absmax / qmax, 1.0).astype(np.float32)
        zero = np.zeros_like(scale)
        codes = np.clip(np.round(grouped / scale), -(qmax + 1), qmax)
    else:
        valid = (np.arange(padded_in) < in_f).reshape(1, n_groups, group_size)
        gmax = np.where(valid, grouped, -np.inf).max(axis=2, keepdims=True)
        gmin = np.where(valid, grouped, np.inf).min(axis=2, keepdims=True)
        gmax = np.where(np.isfinite(gmax), gmax, 0.0).astype(np.float32)
        gmin = np.where(np.isfinite(gmin), gmin, 0.0).astype(np.float32)
        rng = gmax - gmin
        scale = np.where(rng > 0, rng / qmax, 1.0).astype(np.float32)
        zero = np.round(-gmin / scale).astype(np.float32)
        codes = np.clip(np.round(grouped / scale) + zero, 0, qmax)
    scale2 = scale.reshape(out_f, n_groups).astype(np.float32)
    zero2 = zero.reshape(out_f, n_groups).astype(np.float32)
    return {
        "codes_padded": codes.astype(np.int32).reshape(out_f, padded_in),
        "scale": scale2,
        "zero": zero2,
        "scale_f16": scale2.astype(np.float16),
        "zero_f16": zero2.astype(np.float16),
        "bits": bits,
        "symmetric": symmetric,
        "n_groups": n_groups,
        "padded_in": padded_in,
        "shape": (out_f, in_f),
    }


def pack_4bit(codes: Any) -> np.ndarray:
    """Two 4-bit codes per byte, the even column in the low nibble
    (``src/lemoq/quant/pack.py:21-37``)."""
    c = np.asarray(codes).astype(np.int32)
    if c.shape[-1] % 2:
        raise ValueError("last dim must be even")
    return ((c[..., 0::2] & 0xF) | ((c[..., 1::2] & 0xF) << 4)).astype(np.uint8)


def unpack_4bit(packed: Any, signed: bool = True) -> np.ndarray:
    """Inverse of ``pack_4bit`` (``src/lemoq/quant/pack.py:40-63``); ``signed``
    sign-extends -8..7."""
    p = np.asarray(packed).astype(np.int32)
    out = np.stack((p & 0xF, (p >> 4) & 0xF), axis=-1).reshape(p.shape[:-1] + (p.shape[-1] * 2,))
    if signed:
        out = np.where(out >= 8, out - 16, out)
    return out.astype(np.int8 if signed else np.uint8)


def dequant_tile(codes: Any, scale: Any, zero: Any, group_size: int, symmetric: bool,
                 in_features: int | None = None) -> np.ndarray:
    """``_dequant_tile`` of ``src/lemoq/kernels/reference.py:28-47``: codes
    (out, padded) as fp32, ``codes * scale`` or ``(codes - zero) * scale`` per
    group in fp32 (scale and zero converted to fp32 from their stored dtype),
    cut to ``in_features`` columns."""
    c = np.asarray(codes).astype(np.float32)
    rows, padded = c.shape
    ng = padded // group_size
    s = np.asarray(scale).astype(np.float32).reshape(rows, ng, 1)
    g = c.reshape(rows, ng, group_size)
    if symmetric:
        w = g * s
    else:
        w = (g - np.asarray(zero).astype(np.float32).reshape(rows, ng, 1)) * s
    w = w.reshape(rows, padded)
    return w[:, : (padded if in_features is None else in_features)]


E2M1_MAG = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)
MX_BLOCK = 32


def mxfp4_quantize(weight: Any) -> dict[str, Any]:
    """MXFP4 quantiser restated from ``quantize_mxfp4``
    (``src/lemoq/quant/mxfp4.py:50-102``) with the same torch CPU ops: blocks
    of 32 along the input dim (zero padded), ``X = clamp(floor(log2(amax)) - 2,
    -127, 127)`` (-127 for an all-zero block), scale byte ``X + 127``,
    ``v = w / 2^X``, the magnitude code is the argmin (first index on ties) of
    ``|min(|v|, 6) - E2M1_MAG|``, the sign bit ``v < 0``; codes packed two per
    byte, the even column low."""
    import torch  # noqa: PLC0415

    w = torch.as_tensor(weight, dtype=torch.float32)
    if w.ndim != 2:
        raise ValueError("2-D weights only")
    orig_in = int(w.shape[1])
    pad = (-orig_in) % MX_BLOCK
    padded = torch.nn.functional.pad(w, (0, pad))
    out_f, padded_in = padded.shape
    blocks = padded.reshape(out_f, padded_in // MX_BLOCK, MX_BLOCK)
    amax = blocks.abs().amax(dim=-1)
    x = torch.where(amax > 0, torch.floor(torch.log2(amax)) - 2, torch.full_like(amax, -127.0)).clamp(-127, 127)
    scale_bytes = (x + 127).to(torch.uint8)
    scale = torch.exp2(x)
    mags = torch.tensor(E2M1_MAG, dtype=torch.float32)
    norm = blocks / scale.unsqueeze(-1)
    mag = norm.abs().clamp(max=E2M1_MAG[-1])
    idx = (mag.unsqueeze(-1) - mags).abs().argmin(dim=-1)
    codes = (((norm < 0).to(torch.uint8) << 3) | idx.to(torch.uint8)).reshape(out_f, padded_in)
    return {
        "codes": codes.numpy(),
        "codes_packed": pack_4bit(codes.numpy()),
        "scales": scale_bytes.numpy(),
        "orig_in": orig_in,
        "padded_in": int(padded_in),
    }


def mxfp4_dequantize(packed: Any, scales: Any, orig_in: int) -> np.ndarray:
    """``dequantize_packed`` (``src/lemoq/quant/mxfp4.py:105-122``): unsigned
    nibbles, ``E2M1_MAG[c & 7]`` times -1 when ``c & 8``, times
    ``exp2(X - 127)`` in fp32, cut to ``orig_in`` columns."""
    s = np.asarray(scales).astype(np.int64)
    rows, nblk = s.shape
    codes = unpack_4bit(packed, signed=False).astype(np.int64).reshape(rows, nblk * MX_BLOCK)
    mag = np.asarray(E2M1_MAG, dtype=np.float32)[codes & 7]
    sign = np.where((codes & 8) > 0, np.float32(-1.0), np.float32(1.0))
    import torch  # noqa: PLC0415

    # torch's fp32 exp2, as the reference (exact at every integer; numpy's
    # float32 exp2 is one ulp off at 127)
    scale = torch.exp2(torch.from_numpy(s.astype(np.float32)) - 127.0).numpy()
    w = (mag * sign).reshape(rows, nblk, MX_BLOCK) * scale[:, :, None]
    return w.reshape(rows, nblk * MX_BLOCK)[:, :orig_in].astype(np.float32)
