"""Fused RMSNorm with HF rounding points (``lemoq_rmsnorm``).

Replaces ``rms_norm_fused`` (``src/lemoq/kernels/rmsnorm.py:102-163``):
``y = (x * rsqrt(mean(x^2) + eps)).to(fp16) * weight`` — the normalised value is
rounded to fp16 first and the product with the fp16 weight is rounded once
(HF ``OlmoeRMSNorm.forward``), with the mean of squares in fp32.  One block per
row; rows of up to 8192 elements.
"""

from __future__ import annotations

from typing import Any

from lemoq import _hip

__all__ = ["RMSNORM_CONFIG", "rms_norm_fused", "fused_available", "unavailable_reason", "warm"]

RMSNORM_CONFIG: dict[str, int] = {}
MAX_HIDDEN = 8192


def unavailable_reason() -> str | None:
    """Why ``fused_available()`` is False, or None when it is True."""
    return _hip.unavailable_reason()


def fused_available() -> bool:
    try:
        import torch  # noqa: PLC0415

        return _hip.library_available() and bool(torch.cuda.is_available())
    except Exception:  # noqa: BLE001
        return False


def rms_norm_fused(
    x: Any, weight: Any, eps: float, *, out_dtype: Any = None, config: dict[str, Any] | None = None
) -> Any:
    import torch  # noqa: PLC0415

    del config
    if x.dim() < 1:
        raise ValueError("x needs at least one dimension")
    if not x.is_contiguous():
        raise ValueError("x must be contiguous")
    if not weight.is_contiguous():
        raise ValueError("weight must be contiguous")
    if x.dtype != torch.float16:
        raise NotImplementedError("x must be fp16, got %s" % x.dtype)
    if weight.dtype != torch.float16:
        raise NotImplementedError("weight must be fp16, got %s" % weight.dtype)
    H = int(x.shape[-1])
    if int(weight.numel()) != H or weight.dim() != 1:
        raise ValueError("weight must be (H,) with H=%d, got %r" % (H, tuple(weight.shape)))
    if H > MAX_HIDDEN:
        raise NotImplementedError("H=%d exceeds the block limit %d" % (H, MAX_HIDDEN))
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out_dtype not in (torch.float16, torch.float32, torch.float64):
        raise NotImplementedError("out_dtype must be fp16, fp32 or fp64, got %s" % out_dtype)
    _hip.require_rocm(x, weight, what="rms_norm_fused")
    y = torch.empty_like(x)
    M = int(x.numel()) // H if H else 0
    if M:
        _hip.call(
            "lemoq_rmsnorm", _hip.ptr(x), M, H, _hip.ptr(weight), float(eps), _hip.ptr(y),
            _hip.stream_of(x.device),
        )
    # The reference stores the kernel's fp16 product into an out_dtype buffer
    # (src/lemoq/kernels/rmsnorm.py:147-160): a wider dtype holds the same values.
    return y if out_dtype == torch.float16 else y.to(out_dtype)


def warm(x: Any, weight: Any, eps: float, **kwargs: Any) -> None:
    rms_norm_fused(x, weight, eps, **kwargs)
