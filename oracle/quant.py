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
