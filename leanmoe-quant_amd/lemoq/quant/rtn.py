"""Per-group symmetric RTN, 8-bit, on the device (HIP kernel ``lemoq_rtn_quantize_w8``).

Same semantics as the reference's ``lemoq.quant.rtn.quantize_rtn``
(``src/lemoq/quant/rtn.py:38-99``) for ``bits=8, symmetric=True``:
groups of ``group_size`` along the input dimension, the last group
zero-padded; ``scale = absmax/127`` in fp32 (1.0 for an all-zero group);
``codes = round_half_even(w/scale).clamp(-128, 127)``.  The fp16 copy of the
scale is what the packed operators store (``moe_grouped_quant.py:232``,
``linear.py:332``).

Differences from the reference, stated: codes are returned as int8 (the
packed storage type) rather than int32, and only 8-bit symmetric is built
(the 4-bit and asymmetric schemes are outside the decode hot path).
"""

from __future__ import annotations

import math
from typing import Any

from lemoq import _hip


def qmax_for(bits: int, symmetric: bool = True) -> int:
    return (2 ** (bits - 1)) - 1 if symmetric else (2**bits) - 1


def quantize_rtn(
    weight: Any, *, bits: int = 8, group_size: int = 128, symmetric: bool = True
) -> dict[str, Any]:
    """Quantize a 2-D device weight; returns the reference's dict keys.

    ``codes_padded`` (out, padded_in) int8, ``codes`` its ``[:, :in]`` view,
    ``scale`` (out, n_groups) fp32, ``scale_f16`` the fp16 cast, ``zero`` zeros.
    """
    import torch  # noqa: PLC0415

    if not torch.is_tensor(weight):
        raise TypeError("weight must be a tensor")
    if weight.ndim != 2:
        raise ValueError("only 2-D weights are supported, got ndim=%d" % weight.ndim)
    if group_size <= 0:
        raise ValueError("group_size must be > 0")
    if bits not in (4, 8):
        raise ValueError("only 4 and 8 bit are defined, got %r" % (bits,))
    if bits != 8 or not symmetric:
        raise NotImplementedError("the HIP build implements 8-bit symmetric RTN only")
    _hip.require_rocm(weight, what="quantize_rtn")
    w = weight.float().contiguous()
    out_features, in_features = int(w.shape[0]), int(w.shape[1])
    n_groups = int(math.ceil(in_features / group_size))
    padded_in = n_groups * int(group_size)
    codes = torch.empty((out_features, padded_in), dtype=torch.int8, device=w.device)
    scale32 = torch.empty((out_features, n_groups), dtype=torch.float32, device=w.device)
    scale16 = torch.empty((out_features, n_groups), dtype=torch.float16, device=w.device)
    _hip.call(
        "lemoq_rtn_quantize_w8",
        _hip.ptr(w),
        out_features,
        in_features,
        int(group_size),
        _hip.ptr(codes),
        _hip.ptr(scale16),
        _hip.ptr(scale32),
        _hip.stream_of(w.device),
    )
    return {
        "codes": codes[:, :in_features],
        "codes_padded": codes,
        "scale": scale32,
        "scale_f16": scale16,
        "zero": torch.zeros_like(scale32),
        "bits": 8,
        "group_size": int(group_size),
        "symmetric": True,
        "shape": (out_features, in_features),
        "n_groups": n_groups,
        "padded_in": padded_in,
        "device": str(w.device),
    }
