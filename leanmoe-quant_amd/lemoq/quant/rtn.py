"""Per-group RTN at 4 or 8 bits, symmetric or asymmetric, on the device
(HIP kernel ``lemoq_rtn_quantize``).

Same semantics as the reference's ``lemoq.quant.rtn.quantize_rtn``
(``src/lemoq/quant/rtn.py:38-99``): groups of ``group_size`` along the input
dimension, the last group zero-padded; symmetric ``scale = absmax/qmax``
(1.0 for an all-zero group), ``codes = round_half_even(w/scale).clamp(-qmax-1,
qmax)``; asymmetric over the real columns only, ``scale = (max - min)/qmax``,
``zero = round(-min/scale)``, ``codes = (round(w/scale) + zero).clamp(0,
qmax)``.  The fp16 copies of scale and zero are what the packed operators
store (``src/lemoq/quant/linear.py:330-340``, ``moe_grouped_quant.py:232``).

Differences from the reference, stated: codes come back in their storage
types (int8 for 8-bit symmetric, uint8 for 8-bit asymmetric, and for 4 bits
the packed bytes of ``pack.pack_4bit`` plus the unpacked int8 / uint8 codes)
rather than int32.
"""

from __future__ import annotations

import math
from typing import Any

from lemoq import _hip

__all__ = ["qmax_for", "quantize_rtn", "dequantize_rtn", "quantization_error"]


def qmax_for(bits: int, symmetric: bool = True) -> int:
    return (2 ** (bits - 1)) - 1 if symmetric else (2**bits) - 1


def quantize_rtn(
    weight: Any, *, bits: int = 8, group_size: int = 128, symmetric: bool = True
) -> dict[str, Any]:
    """Quantize a 2-D device weight; returns the reference's dict keys.

    ``codes_padded`` (out, padded_in) unpacked codes (int8; uint8 when
    asymmetric), ``codes`` its ``[:, :in]`` view, ``packed`` the storage form
    (``codes_padded`` itself at 8 bits, two codes per byte at 4), ``scale`` /
    ``zero`` (out, n_groups) fp32 and ``scale_f16`` / ``zero_f16`` their fp16
    casts.
    """
    import torch  # noqa: PLC0415

    from lemoq.quant.pack import unpack_4bit  # noqa: PLC0415

    if not torch.is_tensor(weight):
        raise TypeError("weight must be a tensor")
    if weight.ndim != 2:
        raise ValueError("only 2-D weights are supported, got ndim=%d" % weight.ndim)
    if group_size <= 0:
        raise ValueError("group_size must be > 0")
    if bits not in (4, 8):
        raise ValueError("only 4 and 8 bit are defined, got %r" % (bits,))
    if bits == 4 and group_size % 2 != 0:
        raise ValueError("4-bit packing needs an even group_size, got %d" % group_size)
    _hip.require_rocm(weight, what="quantize_rtn")
    w = weight.float().contiguous()
    out_features, in_features = int(w.shape[0]), int(w.shape[1])
    n_groups = int(math.ceil(in_features / group_size))
    padded_in = n_groups * int(group_size)
    dev = w.device
    code_dtype = torch.int8 if (bits == 8 and symmetric) else torch.uint8
    packed = torch.empty((out_features, padded_in if bits == 8 else padded_in // 2), dtype=code_dtype,
                         device=dev)
    scale32 = torch.empty((out_features, n_groups), dtype=torch.float32, device=dev)
    scale16 = torch.empty((out_features, n_groups), dtype=torch.float16, device=dev)
    zero32 = torch.empty((out_features, n_groups), dtype=torch.float32, device=dev)
    zero16 = torch.empty((out_features, n_groups), dtype=torch.float16, device=dev)
    _hip.call(
        "lemoq_rtn_quantize",
        _hip.ptr(w),
        out_features,
        in_features,
        int(group_size),
        int(bits),
        1 if symmetric else 0,
        _hip.ptr(packed),
        _hip.ptr(scale16),
        _hip.ptr(scale32),
        _hip.ptr(zero16),
        _hip.ptr(zero32),
        _hip.stream_of(dev),
    )
    codes = packed if bits == 8 else unpack_4bit(packed, signed=symmetric)
    return {
        "codes": codes[:, :in_features],
        "codes_padded": codes,
        "packed": packed,
        "scale": scale32,
        "scale_f16": scale16,
        "zero": zero32,
        "zero_f16": zero16,
        "bits": int(bits),
        "group_size": int(group_size),
        "symmetric": bool(symmetric),
        "shape": (out_features, in_features),
        "n_groups": n_groups,
        "padded_in": padded_in,
        "device": str(dev),
    }


def dequantize_rtn(q: dict[str, Any], dtype: Any = None) -> Any:
    """Inverse of ``quantize_rtn`` (``src/lemoq/quant/rtn.py:102-114``): fp32
    ``codes * scale`` or ``(codes - zero) * scale`` with the fp32 scale and
    zero, cut to the input width; ``dtype`` rounds the fp32 result once."""
    import torch  # noqa: PLC0415

    from lemoq.quant.formats import dequantize, format_id  # noqa: PLC0415

    w = dequantize(q["packed"], q["scale"], None if q["symmetric"] else q["zero"],
                   fmt=format_id(q["bits"], q["symmetric"]), group_size=q["group_size"], k_out=q["shape"][1],
                   dtype=torch.float32)
    return w.to(dtype) if dtype is not None else w


def quantization_error(weight: Any, q: dict[str, Any]) -> dict[str, float]:
    """Error of a quantisation against its weight (the reference's report,
    ``src/lemoq/quant/rtn.py:117-132``): max and mean absolute error, the max
    relative to the weight's absmax, and the SNR in dB (signal power over error
    power, each floored at 1e-12)."""
    w = weight.float()
    diff = w - dequantize_rtn(q)
    top = float(w.abs().max()) or 1.0
    err_pow = float((diff * diff).mean()) or 1e-12
    sig_pow = float((w * w).mean()) or 1e-12
    return {"max_abs_err": float(diff.abs().max()), "mean_abs_err": float(diff.abs().mean()),
            "max_rel_err_vs_absmax": float(diff.abs().max()) / top,
            "snr_db": 10.0 * math.log10(sig_pow / err_pow)}
