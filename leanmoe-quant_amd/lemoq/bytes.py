"""Byte accounting of one batch-1 decode step (the roofline numerator).

Restates the reference's byte model (``benchmarks/bytes.py:182-411``:
``weight_budget`` = ``[W]``, ``kv_budget``, ``byte_budget`` = ``[T]``,
``attainments``) for the decode path this package runs:

* ``[W]`` counts the weights one token streams: q|k|v and o projections of
  every layer, the fp16 router, the top-k experts' gate/up and down
  projections, and lm_head.  A w8 matrix of ``rows x in_f`` costs
  ``rows*in_f`` code bytes plus ``rows*ceil(in_f/group)`` fp16 scales (groups
  run along the input dimension, one set per row).  The embedding row (one
  gather) and the RMSNorm weights are streamed too but, as in the
  reference, are reported outside ``[W]``.
* KV read bytes per step: every layer reads K and V for ``filled`` tokens;
  fp16 costs ``2*heads*D*2`` bytes per token and layer, KV-INT8 costs
  ``2*heads*(D + 2)`` (int8 codes plus one fp16 scale per head and token).
  (The reference's payload still counts KV-INT8 as fp16; this model counts
  what is read.)
* ``attainment = bytes / seconds / bandwidth``.
* 4-bit weights (the w4a16 cell: attention and experts at 4 bits, router and
  lm_head fp16) cost ``rows*in_f/2`` code bytes plus the same scales.

Pinned by the reference's anchors (tests/test_bytes.py:39-79 of LeanMoE-Quant):
fp16 ``[W]`` = 2,357,723,136 B; fp16 KV read = 134,217,728 B at ctx 1024 and
536,870,912 B at ctx 4096; w8 attention + experts with fp16 lm_head =
1,300,758,528 B (EXP-p4c-01-in-graph-attention.md:152).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

__all__ = ["WeightBits", "weight_budget", "kv_read_bytes", "step_bytes", "attainment"]


@dataclass(frozen=True)
class WeightBits:
    """Storage of each weight family: 16 (fp16), or 8 / 4 (codes + fp16 group scales;
    4-bit codes two per byte)."""

    attention: int = 8
    experts: int = 8
    lm_head: int = 8
    router: int = 16
    group_size: int = 128


def _matrix_bytes(rows: int, in_f: int, bits: int, group: int) -> int:
    """fp16 bytes, or packed codes (``params * bits // 8``) plus one fp16 scale per
    row and group along the input dimension (the reference's ``_quantized_bytes``,
    ``benchmarks/bytes.py:141-171``)."""
    if bits == 16:
        return rows * in_f * 2
    if bits in (4, 8):
        return rows * in_f * bits // 8 + rows * (-(-in_f // group)) * 2
    raise ValueError("bits must be 4, 8 or 16, got %r" % (bits,))


def weight_budget(shape: Any, bits: WeightBits | None = None) -> dict[str, Any]:
    """``[W]`` of one decode token for an OLMoE-style ``shape`` (fields hidden, heads,
    head_dim, layers, num_experts, top_k, ffn, vocab; MHA)."""
    b = bits or WeightBits()
    g = b.group_size
    L, H, HD = shape.layers, shape.hidden, shape.heads * shape.head_dim
    F, E, K, V = shape.ffn, shape.num_experts, shape.top_k, shape.vocab
    items = [
        ("attention", L * (_matrix_bytes(3 * HD, H, b.attention, g) + _matrix_bytes(H, HD, b.attention, g))),
        ("router", L * _matrix_bytes(E, H, b.router, g)),
        ("experts(top-k)", L * K * (_matrix_bytes(2 * F, H, b.experts, g) + _matrix_bytes(H, F, b.experts, g))),
        ("lm_head", _matrix_bytes(V, H, b.lm_head, g)),
    ]
    total = sum(v for _, v in items)
    out_items = [
        {"name": n, "bytes": v, "share_pct": 100.0 * v / total, "counted_in_total": True} for n, v in items
    ]
    norms = (L * (2 * H + 2 * HD) + H) * 2
    out_items.append({"name": "norm_weights", "bytes": norms, "share_pct": None, "counted_in_total": False})
    out_items.append({"name": "embedding_row", "bytes": H * 2, "share_pct": None, "counted_in_total": False})
    return {"total_bytes": total, "items": out_items, "streamed_bytes": total + norms + H * 2}


def kv_read_bytes(shape: Any, filled: int, *, kv: str = "int8", batch: int = 1) -> int:
    """K+V bytes read by the attention of all layers for ``filled`` cached tokens."""
    if filled < 0 or batch < 1:
        raise ValueError("filled must be >= 0 and batch >= 1")
    per_token_layer = {
        "fp16": 2 * shape.heads * shape.head_dim * 2,
        "int8": 2 * shape.heads * (shape.head_dim + 2),
    }
    if kv not in per_token_layer:
        raise ValueError("kv must be 'int8' or 'fp16', got %r" % (kv,))
    return batch * shape.layers * filled * per_token_layer[kv]


def step_bytes(shape: Any, filled: int, *, bits: WeightBits | None = None, kv: str = "int8") -> int:
    """HBM bytes one decode step must move: streamed weights (``[W]`` + norm weights +
    embedding row) plus the KV read at ``filled`` tokens."""
    return weight_budget(shape, bits)["streamed_bytes"] + kv_read_bytes(shape, filled, kv=kv)


def attainment(nbytes: float, seconds: float, bandwidth_bytes_per_s: float) -> float:
    """Fraction of the bandwidth roofline reached: ``bytes / seconds / bandwidth``."""
    if seconds <= 0 or bandwidth_bytes_per_s <= 0:
        raise ValueError("seconds and bandwidth must be positive")
    return nbytes / seconds / bandwidth_bytes_per_s
