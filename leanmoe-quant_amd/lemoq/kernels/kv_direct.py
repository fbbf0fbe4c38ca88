"""Bitwise write of the new fp16 k/v rows into a static cache slot (``lemoq_kv_write_f16``).

Replaces ``kv_direct_write`` / ``kv_direct_write_applicable`` of the reference
(``src/lemoq/kernels/kv_direct.py:37-137``) with the slot contract of
``kv_write.write_kv_slot`` (``src/lemoq/kernels/kv_write.py:26-50``): the layer's
``keys``/``values`` buffers ``(1, H, S, D)`` keep their addresses, only slot
``pos`` changes, and ``pos`` is read on the device (graph-safe).
"""

from __future__ import annotations

from typing import Any

from lemoq import _hip

__all__ = ["kv_direct_write", "kv_direct_write_applicable"]


def kv_direct_write_applicable(cache_layer: Any, key_states: Any, value_states: Any) -> bool:
    import torch  # noqa: PLC0415

    if not (torch.is_tensor(key_states) and torch.is_tensor(value_states)):
        return False
    if not (key_states.is_cuda and value_states.is_cuda):
        return False
    keys = getattr(cache_layer, "keys", None)
    values = getattr(cache_layer, "values", None)
    if keys is None or values is None:
        return False
    if not (keys.is_cuda and values.is_cuda):
        return False
    if keys.shape != values.shape or keys.dim() != 4 or keys.shape[0] != 1:
        return False
    if not (keys.is_contiguous() and values.is_contiguous()):
        return False
    if key_states.dtype is not keys.dtype or value_states.dtype is not values.dtype:
        return False
    if keys.dtype is not torch.float16:
        return False
    _, heads, _, dim = keys.shape
    if key_states.shape != (1, heads, 1, dim) or value_states.shape != (1, heads, 1, dim):
        return False
    if key_states.stride(-1) != 1 or value_states.stride(-1) != 1:
        return False
    if key_states.stride(1) != value_states.stride(1):
        return False
    return dim >= 2 and (dim & (dim - 1)) == 0


def kv_direct_write(layer: Any, key_states: Any, value_states: Any, cache_position: Any) -> None:
    """Copy (1,H,1,D) k/v into ``layer.keys/values[:, :, pos]``; ``pos`` a device int64."""
    import torch  # noqa: PLC0415

    if not kv_direct_write_applicable(layer, key_states, value_states):
        raise RuntimeError("kv_direct_write: shape/layout guard failed (see kv_direct_write_applicable)")
    pos = cache_position
    if not torch.is_tensor(pos) or pos.numel() != 1 or pos.dtype != torch.int64:
        raise ValueError("cache_position must be a one-element int64 device tensor (decode)")
    _hip.require_rocm(pos, what="kv_direct_write")
    _, heads, max_len, dim = layer.keys.shape
    _hip.call(
        "lemoq_kv_write_f16",
        _hip.ptr(key_states), _hip.ptr(value_states), int(key_states.stride(1)),
        _hip.ptr(layer.keys), _hip.ptr(layer.values), int(max_len) * int(dim),
        _hip.ptr(pos.reshape(1)), int(heads), int(dim), _hip.stream_of(key_states.device),
    )
