"""MXFP4 (OCP MX v1.0) weights: E2M1 codes with one E8M0 power-of-two scale
per block of 32, quantised and dequantised on the device.

Same format and semantics as the reference's host-side module
(``src/lemoq/quant/mxfp4.py:1-129``):

- a block of 32 elements along the input dim shares one E8M0 byte, value
  ``2^(X - 127)`` (bias 127, no inf / NaN encodings);
- ``X = floor(log2(amax)) - 2`` (E2M1's largest normal is 6 = 1.5 * 2^2),
  clamped to [-127, 127]; an all-zero block stores byte 0 and all-zero codes;
- E2M1: bit 3 the sign, bits 2..0 the magnitude code of
  {0, 0.5, 1, 1.5, 2, 3, 4, 6}; round to nearest, ties to the smaller
  magnitude; values beyond 6 * scale saturate to +-6 (a known wart of the
  format, kept);
- codes pack two per byte, the even column in the low nibble
  (``lemoq.quant.pack``).

``quantize_mxfp4`` runs ``lemoq_mxfp4_quantize``; ``dequantize_packed`` runs
``lemoq_dequant_q`` with ``LEMOQ_QFMT_MXFP4``.
"""

from __future__ import annotations

from typing import Any

from lemoq import _hip

__all__ = ["BLOCK", "e2m1_decode", "e8m0_to_scale", "quantize_mxfp4", "dequantize_packed", "dequantize_mxfp4"]

_E2M1_MAG = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)  # magnitude codes 0..7
_EMAX_ELEM = 2  # E2M1: 6 = 1.5 * 2^2
BLOCK = 32
_E8M0_BIAS = 127


def e2m1_decode(code: int) -> float:
    """4-bit E2M1 code (bit 3 sign, bits 2..0 magnitude) -> value."""
    mag = _E2M1_MAG[code & 0x7]
    return -mag if (code & 0x8) else mag


def e8m0_to_scale(byte: int) -> float:
    """E8M0 byte -> 2^(byte - 127) (byte 0 is 2^-127, the all-zero block's placeholder)."""
    return 2.0 ** (byte - _E8M0_BIAS)


def quantize_mxfp4(weight: Any, *, block: int = BLOCK) -> dict[str, Any]:
    """Device weight (out, in) -> {"codes_packed": uint8 (out, padded_in/2),
    "scales": uint8 (out, padded_in/32), "orig_in", "padded_in", "block"}."""
    import torch  # noqa: PLC0415

    if block != BLOCK:
        raise ValueError("the MXFP4 block is fixed at 32 (OCP MX), got %d" % block)
    if weight.ndim != 2:
        raise ValueError("only 2-D weights are supported, got ndim=%d" % weight.ndim)
    _hip.require_rocm(weight, what="quantize_mxfp4")
    w = weight.float().contiguous()
    out_features, orig_in = int(w.shape[0]), int(w.shape[1])
    nblk = -(-orig_in // BLOCK)
    codes = torch.empty((out_features, nblk * BLOCK // 2), dtype=torch.uint8, device=w.device)
    scales = torch.empty((out_features, nblk), dtype=torch.uint8, device=w.device)
    _hip.call("lemoq_mxfp4_quantize", _hip.ptr(w), out_features, orig_in, _hip.ptr(codes), _hip.ptr(scales),
              _hip.stream_of(w.device))
    return {"codes_packed": codes, "scales": scales, "orig_in": orig_in, "padded_in": nblk * BLOCK,
            "block": BLOCK}


def dequantize_packed(packed: Any, scales: Any, orig_in: int, *, block: int = BLOCK, dtype: Any = None) -> Any:
    """Packed codes + E8M0 bytes -> (out, orig_in) weights: ``e2m1(c) * 2^(X - 127)``
    in fp32, rounded once to ``dtype`` when given."""
    import torch  # noqa: PLC0415

    from lemoq.quant.formats import QFMT_MXFP4, dequantize  # noqa: PLC0415

    if block != BLOCK:
        raise ValueError("the MXFP4 block is fixed at 32 (OCP MX), got %d" % block)
    if scales.dtype != torch.uint8:
        raise ValueError("MXFP4 scales must be uint8 E8M0 bytes, got %s" % scales.dtype)
    out = dtype if dtype in (torch.float16, torch.float32) else torch.float32
    w = dequantize(packed.contiguous(), scales.contiguous(), None, fmt=QFMT_MXFP4, group_size=BLOCK,
                   k_out=int(orig_in), dtype=out)
    return w if dtype is None or dtype == out else w.to(dtype)


def dequantize_mxfp4(q: dict[str, Any], *, dtype: Any = None) -> Any:
    """``dequantize_packed`` of a ``quantize_mxfp4`` result."""
    return dequantize_packed(q["codes_packed"], q["scales"], q["orig_in"], block=q["block"], dtype=dtype)
