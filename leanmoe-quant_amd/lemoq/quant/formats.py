"""Weight formats of the dense dequant operator and their HIP dequantisation.

Format ids match ``LEMOQ_QFMT_*`` of ``include/lemoq_hip.h``.  The reference
selects them with the ``bits`` / ``symmetric`` / ``mxfp4`` arguments of
``dequant_gemm_fused`` (``src/lemoq/kernels/_dequant_triton.py:155-293``) and
the schemes of ``QuantLinear`` (``src/lemoq/quant/linear.py:76-89``):

=============  ============================  ==========================
format         codes (N, P)                  w
=============  ============================  ==========================
W8             int8, P = padded_in           c * s
W8_ASYM        uint8, P = padded_in          (c - z) * s
W4             packed int4, P = padded_in/2  c * s
W4_ASYM        packed uint4, P = padded_in/2 (c - z) * s
MXFP4          packed E2M1, P = padded_in/2  e2m1(c) * 2^(X - 127)
=============  ============================  ==========================
"""

from __future__ import annotations

from typing import Any

from lemoq import _hip

__all__ = ["QFMT_W8", "QFMT_W8_ASYM", "QFMT_W4", "QFMT_W4_ASYM", "QFMT_MXFP4", "format_id", "dequantize"]

QFMT_W8, QFMT_W8_ASYM, QFMT_W4, QFMT_W4_ASYM, QFMT_MXFP4 = range(5)


def format_id(bits: int, symmetric: bool, mxfp4: bool = False) -> int:
    if mxfp4:
        return QFMT_MXFP4
    if bits == 8:
        return QFMT_W8 if symmetric else QFMT_W8_ASYM
    if bits == 4:
        return QFMT_W4 if symmetric else QFMT_W4_ASYM
    raise NotImplementedError("4- and 8-bit formats only, got %r" % (bits,))


def scale_zero_args(scale: Any, zero: Any) -> tuple[Any, Any, int]:
    """Scale and zero point of one common float type (an fp16 one is widened to
    fp32, which is exact, when the other is fp32); returns them and the
    scale_is_f32 flag of the C-ABI.  uint8 (E8M0) scales pass through."""
    import torch  # noqa: PLC0415

    if scale.dtype == torch.uint8:
        return scale, zero, 0
    if scale.dtype not in (torch.float16, torch.float32):
        raise ValueError("scale must be fp16 or fp32, got %s" % scale.dtype)
    if zero is not None and zero.dtype not in (torch.float16, torch.float32):
        raise ValueError("zero must be fp16 or fp32, got %s" % zero.dtype)
    wide = scale.dtype == torch.float32 or (zero is not None and zero.dtype == torch.float32)
    if wide:
        scale = scale.float().contiguous()
        zero = None if zero is None else zero.float().contiguous()
    return scale, zero, 1 if wide else 0


def dequantize(qweight: Any, scale: Any, zero: Any, *, fmt: int, group_size: int, k_out: int,
               dtype: Any = None) -> Any:
    """Dense (N, k_out) weight of a packed weight (``lemoq_dequant_q``): fp32
    arithmetic as the reference's separate arm, stored as fp32 or rounded once
    to fp16 (``dtype``; fp32 when None)."""
    import torch  # noqa: PLC0415

    dtype = torch.float32 if dtype is None else dtype
    if dtype not in (torch.float32, torch.float16):
        raise NotImplementedError("dequantised weights are fp32 or fp16, got %s" % dtype)
    N = int(qweight.shape[0])
    n_groups = int(scale.shape[1])
    padded_in = n_groups * int(group_size)
    scale, zero, s32 = scale_zero_args(scale, zero)
    _hip.require_rocm(qweight, scale, what="dequantize")
    w = torch.empty((N, int(k_out)), dtype=dtype, device=qweight.device)
    if N == 0:
        return w
    _hip.call("lemoq_dequant_q", _hip.ptr(qweight), int(fmt), _hip.ptr(scale),
              _hip.ptr(zero) if zero is not None else None, s32, N, padded_in, int(group_size), _hip.ptr(w),
              int(k_out), int(k_out), 1 if dtype == torch.float32 else 0, _hip.stream_of(qweight.device))
    return w
