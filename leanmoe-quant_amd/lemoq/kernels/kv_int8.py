"""KV-INT8 cache: per-token symmetric int8 quantisation written on the device.

Operator surface of the reference's ``src/lemoq/kernels/kv_int8.py``:
``kv_int8_rows_applicable`` (``:64-95``), ``kv_int8_bulk_quantize``
(``:127-163``), ``kv_int8_init_buffers`` (``:166-170``),
``kv_int8_cache_write`` (``:223-257``), ``kv_int8_write`` (``:318-355``) and the
per-row quantiser ``quantize_per_token_int8`` (``:30-41``) — all computed by
the HIP kernels ``lemoq_kv_write_i8`` / ``lemoq_kv_quantize_rows``.

Arithmetic (bit-exact with the reference's torch math): fp32 ``amax`` of the
row; ``s = amax/127`` correctly rounded (1.0 for an all-zero row);
``code = round_half_even(x/s)`` clamped to [-127, 127]; the scale is stored as
``fp16(s)``.  Unfilled cache slots are codes 0 / scale 1.0.
"""

from __future__ import annotations

from typing import Any

from lemoq import _hip

__all__ = [
    "kv_int8_bulk_quantize",
    "kv_int8_cache_write",
    "kv_int8_init_buffers",
    "kv_int8_rows_applicable",
    "kv_int8_write",
    "quantize_per_token_int8",
]


def _row_guard_failure(k_new: Any, v_new: Any) -> str | None:
    """The first rule that the k/v rows break, or None when the int8 write path
    takes them: two ROCm-resident fp16 tensors of one (1, H, 1, D) shape, both
    contiguous, with D a power of two (the per-row reduction of the kernel)."""
    import torch  # noqa: PLC0415

    pair = (k_new, v_new)
    if not all(torch.is_tensor(t) for t in pair):
        return "k/v are not tensors"
    if not all(t.is_cuda for t in pair):
        return "k/v are not on the GPU"
    if any(t.dtype is not torch.float16 for t in pair):
        return "k/v are not fp16"
    shape = tuple(k_new.shape)
    if tuple(v_new.shape) != shape or len(shape) != 4 or shape[0] != 1 or shape[2] != 1:
        return "k/v are not one (1, H, 1, D) shape"
    if not all(t.is_contiguous() for t in pair):
        return "k/v are not contiguous"
    d = shape[3]
    if d < 1 or d & (d - 1):
        return "head_dim %d is not a power of two" % d
    return None


def kv_int8_rows_applicable(k_new: Any, v_new: Any) -> bool:
    """Row guard of the write path; callers fall back to the fp16 write when False."""
    return _row_guard_failure(k_new, v_new) is None


def _require_rows(k_new: Any, v_new: Any, what: str) -> None:
    why = _row_guard_failure(k_new, v_new)
    if why is not None:
        raise RuntimeError("%s: row guard failed (%s); check kv_int8_rows_applicable first" % (what, why))


def quantize_per_token_int8(x: Any) -> tuple[Any, Any]:
    """``(..., D)`` fp16 device tensor -> ``(codes int8 (..., D), scale fp16 (...))``."""
    import torch  # noqa: PLC0415

    if not torch.is_tensor(x) or x.dim() < 1:
        raise ValueError("x must be a tensor with a last (head_dim) dimension")
    if x.dtype != torch.float16:
        raise NotImplementedError("the HIP quantiser takes fp16 rows, got %s" % x.dtype)
    _hip.require_rocm(x, what="quantize_per_token_int8")
    d = int(x.shape[-1])
    xc = x.contiguous()
    rows = int(xc.numel()) // d if d else 0
    codes = torch.empty(tuple(x.shape), dtype=torch.int8, device=x.device)
    scales = torch.empty(tuple(x.shape[:-1]), dtype=torch.float16, device=x.device)
    if rows:
        _hip.call(
            "lemoq_kv_quantize_rows",
            _hip.ptr(xc), rows, d, _hip.ptr(codes), _hip.ptr(scales), _hip.stream_of(x.device),
        )
    return codes, scales


def kv_int8_bulk_quantize(cache_keys: Any, cache_values: Any, filled: Any = None) -> dict[str, Any]:
    """Quantize fp16 caches ``(1,H,S,D)`` -> ``{kc, ks, vc, vs}``; slots >= filled get 0 / 1.0."""
    import torch  # noqa: PLC0415

    _hip.require_rocm(cache_keys, cache_values, what="kv_int8_bulk_quantize")
    if cache_keys.dim() != 4 or cache_keys.shape != cache_values.shape or cache_keys.shape[0] != 1:
        raise ValueError("caches must be (1,H,S,D) and equal-shaped")
    H, S, D = int(cache_keys.shape[1]), int(cache_keys.shape[2]), int(cache_keys.shape[3])
    if filled is not None:
        filled = int(filled.item()) if hasattr(filled, "item") else int(filled)
        filled = max(0, min(filled, S))
    out: dict[str, Any] = {}
    st = _hip.stream_of(cache_keys.device)
    for name, tensor in (("kc", cache_keys), ("vc", cache_values)):
        codes = torch.zeros((1, H, S, D), dtype=torch.int8, device=tensor.device)
        scales = torch.ones((1, H, S), dtype=torch.float16, device=tensor.device)
        n = S if filled is None else filled
        if n > 0:
            src = tensor[0, :, :n, :].contiguous()  # (H, n, D)
            c = torch.empty((H, n, D), dtype=torch.int8, device=tensor.device)
            s = torch.empty((H, n), dtype=torch.float16, device=tensor.device)
            _hip.call("lemoq_kv_quantize_rows", _hip.ptr(src), H * n, D, _hip.ptr(c), _hip.ptr(s), st)
            codes[0, :, :n, :] = c
            scales[0, :, :n] = s
        out[name] = codes
        out[name.replace("c", "s")] = scales
    return out


def kv_int8_init_buffers(layer_keys: Any, layer_values: Any, filled: Any = None) -> dict[str, Any]:
    """A layer's int8 mirror of its fp16 cache, marked ``initialized``."""
    return {**kv_int8_bulk_quantize(layer_keys, layer_values, filled), "initialized": True}


def kv_int8_cache_write(bufs: dict[str, Any], k_new: Any, v_new: Any, pos: Any) -> None:
    """Quantize the new (1,H,1,D) k/v rows into slot ``pos`` (device int64 tensor)."""
    import torch  # noqa: PLC0415

    _require_rows(k_new, v_new, "kv_int8_cache_write")
    kc = bufs["kc"]
    if (
        kc.dim() != 4
        or kc.shape[1] != k_new.shape[1]
        or kc.shape[3] != k_new.shape[3]
        or kc.shape[0] != 1
        or not kc.is_contiguous()
    ):
        raise RuntimeError(
            "kv_int8_cache_write: buffer shape/layout %s does not match rows %s"
            % (tuple(kc.shape), tuple(k_new.shape))
        )
    if not torch.is_tensor(pos) or pos.numel() != 1 or pos.dtype != torch.int64:
        raise ValueError("pos must be a one-element int64 device tensor")
    _hip.require_rocm(pos, kc, bufs["ks"], bufs["vc"], bufs["vs"], what="kv_int8_cache_write")
    S = int(kc.shape[2])
    _hip.call(
        "lemoq_kv_write_i8",
        _hip.ptr(k_new), _hip.ptr(v_new), int(k_new.shape[1]), int(k_new.shape[3]),
        _hip.ptr(kc), _hip.ptr(bufs["ks"]), _hip.ptr(bufs["vc"]), _hip.ptr(bufs["vs"]),
        int(kc.stride(1)), S, _hip.ptr(pos.reshape(1)), _hip.stream_of(k_new.device),
    )


def kv_int8_write(
    k_new: Any,
    v_new: Any,
    *,
    k_codes: Any = None,
    k_scale: Any = None,
    v_codes: Any = None,
    v_scale: Any = None,
) -> tuple[Any, Any, Any, Any]:
    """Quantize (1,H,1,D) k/v rows into (1,H,1,D) int8 codes + (1,H,1) fp16 scales."""
    import torch  # noqa: PLC0415

    _require_rows(k_new, v_new, "kv_int8_write")
    heads, dim = int(k_new.shape[1]), int(k_new.shape[-1])
    given = (k_codes, k_scale, v_codes, v_scale)
    if all(t is None for t in given):
        # one allocation each for the codes and the scales of both rows
        codes = torch.empty((2, 1, heads, 1, dim), dtype=torch.int8, device=k_new.device)
        scales = torch.empty((2, 1, heads, 1), dtype=torch.float16, device=k_new.device)
        k_codes, v_codes = codes.unbind(0)
        k_scale, v_scale = scales.unbind(0)
    elif any(t is None for t in given):
        raise ValueError("kv_int8_write: pass all four outputs or none")
    _hip.require_rocm(k_codes, k_scale, v_codes, v_scale, what="kv_int8_write")
    _hip.call(
        "lemoq_kv_write_i8",
        _hip.ptr(k_new), _hip.ptr(v_new), heads, dim,
        _hip.ptr(k_codes), _hip.ptr(k_scale), _hip.ptr(v_codes), _hip.ptr(v_scale),
        dim, 1, None, _hip.stream_of(k_new.device),
    )
    return k_codes, k_scale, v_codes, v_scale
