"""w8 dense GEMV with in-register dequantisation (``lemoq_gemv_w8``), and the
multi-token w8 / fp16 linears on the matrix cores (``lemoq_gemm_w8``,
``lemoq_gemm_f16``).

Replaces ``dequant_gemm_fused`` of the reference
(``src/lemoq/kernels/_dequant_triton.py:155-293``) for the branch the decode
hot path uses: 8-bit symmetric codes (int8), fp16 per-group scales along the
input dimension, ``zero=None``.  Same contract: ``y = x @ dequant(qweight).T``
with fp32 accumulation and a single rounding to ``out_dtype`` (fp32 by
default), contiguous inputs required, boundaries raise instead of computing
something wrong.  The 4-bit, asymmetric and MXFP4 branches are outside the
decode path and raise ``NotImplementedError``.
"""

from __future__ import annotations

from typing import Any

from lemoq import _hip

__all__ = ["DEQUANT_GEMM_CONFIGS", "dequant_gemm_fused", "dequant_gemm_separate", "linear_f16",
           "fused_available", "warm"]

# The HIP kernel's tiling is chosen inside the library from N (rows per wave)
# and K (1 KB chunks per row); no tunables are exposed.  Kept for call-site
# compatibility with the reference's `config=` argument.
DEQUANT_GEMM_CONFIGS: dict[str, dict[str, int]] = {"dequant_gemm": {}}

MAX_PADDED_K = 8192


def fused_available() -> bool:
    """True when the HIP library is built and a ROCm device is visible (never raises)."""
    try:
        import torch  # noqa: PLC0415

        return _hip.library_available() and bool(torch.cuda.is_available())
    except Exception:  # noqa: BLE001
        return False


def dequant_gemm_fused(
    x: Any,
    qweight: Any,
    scale: Any,
    zero: Any = None,
    *,
    group_size: int,
    bits: int | None = None,
    symmetric: bool = True,
    out_dtype: Any = None,
    config: dict[str, Any] | None = None,
    mxfp4: bool = False,
) -> Any:
    """``y (M, N) = x (M, K) @ dequant(qweight (N, P), scale (N, n_groups)).T``."""
    import torch  # noqa: PLC0415

    del config
    if x.dim() != 2:
        raise ValueError("x must be 2-D (M, K), got %r" % (tuple(x.shape),))
    if qweight.dim() != 2:
        raise ValueError("qweight must be 2-D (N, P), got %r" % (tuple(qweight.shape),))
    if scale.dim() != 2:
        raise ValueError("scale must be 2-D (N, n_groups), got %r" % (tuple(scale.shape),))
    M, K = int(x.shape[0]), int(x.shape[1])
    N, packed_in = int(qweight.shape[0]), int(qweight.shape[1])
    n_groups = int(scale.shape[1])
    if int(scale.shape[0]) != N:
        raise ValueError("scale has %d rows, qweight has %d" % (int(scale.shape[0]), N))
    if bits is None:
        bits = 4 if qweight.dtype == torch.uint8 else 8
    bits = int(bits)
    if bits not in (4, 8):
        raise NotImplementedError("fused dequant-GEMM implements 4/8-bit, got %d" % bits)
    if mxfp4 or bits != 8 or not symmetric or zero is not None:
        raise NotImplementedError(
            "the HIP build implements the 8-bit symmetric (zero=None) branch only"
        )
    padded_in = n_groups * int(group_size)
    if packed_in != padded_in:
        raise ValueError(
            "qweight width %d != n_groups*group_size %d" % (packed_in, padded_in)
        )
    if K > padded_in:
        raise ValueError("K=%d exceeds padded_in=%d" % (K, padded_in))
    if qweight.dtype != torch.int8:
        raise ValueError("8-bit symmetric qweight must be int8, got %s" % qweight.dtype)
    if x.dtype != torch.float16:
        raise NotImplementedError("x must be fp16 (the w8a16 path), got %s" % x.dtype)
    if scale.dtype != torch.float16:
        raise NotImplementedError("scale must be fp16, got %s" % scale.dtype)
    if out_dtype is None:
        out_dtype = torch.float32
    if out_dtype not in (torch.float32, torch.float16):
        raise NotImplementedError("out_dtype must be fp32 or fp16, got %s" % out_dtype)
    for name, tensor in (("x", x), ("qweight", qweight), ("scale", scale)):
        if not tensor.is_contiguous():
            raise ValueError("%s must be contiguous" % name)
    if int(group_size) % 16 != 0 or padded_in % 16 != 0 or padded_in > MAX_PADDED_K:
        raise NotImplementedError(
            "HIP GEMV needs group_size %% 16 == 0 and padded_in <= %d (got group %d, padded %d)"
            % (MAX_PADDED_K, int(group_size), padded_in)
        )
    _hip.require_rocm(x, qweight, scale, what="dequant_gemm_fused")
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    if M == 0 or N == 0:
        return y
    _hip.call(
        "lemoq_gemv_w8",
        _hip.ptr(x),
        M,
        K,
        _hip.ptr(qweight),
        _hip.ptr(scale),
        N,
        padded_in,
        int(group_size),
        _hip.ptr(y),
        1 if out_dtype == torch.float16 else 0,
        _hip.stream_of(x.device),
    )
    return y


def warm(x: Any, qweight: Any, scale: Any, zero: Any = None, **kwargs: Any) -> None:
    """One real launch (kept for call-site compatibility; HIP code needs no JIT)."""
    dequant_gemm_fused(x, qweight, scale, zero, **kwargs)


def _check_rows(x: Any, K: int, what: str) -> None:
    import torch  # noqa: PLC0415

    if x.dim() != 2 or int(x.shape[1]) != K:
        raise ValueError("%s: x must be (M, %d), got %r" % (what, K, tuple(x.shape)))
    if x.dtype != torch.float16:
        raise NotImplementedError("%s: x must be fp16, got %s" % (what, x.dtype))
    if not x.is_contiguous():
        raise ValueError("%s: x must be contiguous" % what)


def dequant_gemm_separate(
    x: Any,
    qweight: Any,
    scale: Any,
    zero: Any = None,
    *,
    group_size: int,
    bits: int = 8,
    symmetric: bool = True,
    residual: Any = None,
) -> Any:
    """``y (M, N) = fp16(x @ fp16(dequant(qweight)).T)`` on the matrix cores.

    The numerics of the reference's multi-token ``QuantLinear`` arm
    (``dequantized_weight(dtype=fp16)`` then ``F.linear``,
    ``src/lemoq/quant/linear.py:365-395,471-480``) without materialising the
    weight: each code is dequantised to ``fp16(code * scale)`` in registers,
    products accumulate in fp32, the output is rounded to fp16 once.  With
    ``residual`` (M, N) fp16, ``y = fp16(y + residual)``.  K must equal the
    padded width (a multiple of 64 and of ``group_size``).
    """
    import torch  # noqa: PLC0415

    if bits != 8 or not symmetric or zero is not None:
        raise NotImplementedError("the HIP build implements the 8-bit symmetric (zero=None) branch only")
    if qweight.dim() != 2 or qweight.dtype != torch.int8 or not qweight.is_contiguous():
        raise ValueError("qweight must be contiguous int8 (N, K)")
    N, K = int(qweight.shape[0]), int(qweight.shape[1])
    g = int(group_size)
    if scale.dtype != torch.float16 or tuple(scale.shape) != (N, K // max(g, 1)) or not scale.is_contiguous():
        raise ValueError("scale must be contiguous fp16 (N, K/group), got %r" % (tuple(scale.shape),))
    if g <= 0 or g % 64 != 0 or K % g != 0:
        raise NotImplementedError("the matrix-core GEMM needs group_size % 64 == 0 and K % group_size == 0")
    _check_rows(x, K, "dequant_gemm_separate")
    M = int(x.shape[0])
    y = torch.empty((M, N), dtype=torch.float16, device=x.device)
    if residual is not None and (tuple(residual.shape) != (M, N) or residual.dtype != torch.float16
                                 or not residual.is_contiguous()):
        raise ValueError("residual must be contiguous fp16 (M, N)")
    _hip.require_rocm(x, qweight, scale, what="dequant_gemm_separate")
    if M == 0 or N == 0:
        return y
    _hip.call("lemoq_gemm_w8", _hip.ptr(x), M, K, K, None, _hip.ptr(qweight), _hip.ptr(scale), N, g,
              _hip.ptr(y), N, _hip.ptr(residual) if residual is not None else None, N,
              _hip.stream_of(x.device))
    return y


def linear_f16(x: Any, weight: Any, *, splits: int = 1) -> Any:
    """``fp16(x (M, K) @ weight (N, K).T)`` with fp32 accumulation (``F.linear`` in fp16).

    ``splits`` > 1 cuts K into that many ranges summed in order (``lemoq_gemm_f16_splitk``):
    more blocks for narrow outputs such as the 64-expert router."""
    import torch  # noqa: PLC0415

    if weight.dim() != 2 or weight.dtype != torch.float16 or not weight.is_contiguous():
        raise ValueError("weight must be contiguous fp16 (N, K)")
    N, K = int(weight.shape[0]), int(weight.shape[1])
    if K % 64 != 0:
        raise NotImplementedError("linear_f16 needs K % 64 == 0, got %d" % K)
    _check_rows(x, K, "linear_f16")
    M = int(x.shape[0])
    y = torch.empty((M, N), dtype=torch.float16, device=x.device)
    _hip.require_rocm(x, weight, what="linear_f16")
    if M == 0 or N == 0:
        return y
    if splits > 1:
        if K % (64 * splits) != 0:
            raise ValueError("K=%d is not a multiple of 64 * splits (%d)" % (K, splits))
        ws = torch.empty((splits, M, N), dtype=torch.float32, device=x.device)
        _hip.call("lemoq_gemm_f16_splitk", _hip.ptr(x), M, K, K, _hip.ptr(weight), N, _hip.ptr(y), N, int(splits),
                  _hip.ptr(ws), _hip.stream_of(x.device))
        return y
    _hip.call("lemoq_gemm_f16", _hip.ptr(x), M, K, K, _hip.ptr(weight), N, _hip.ptr(y), N,
              _hip.stream_of(x.device))
    return y
