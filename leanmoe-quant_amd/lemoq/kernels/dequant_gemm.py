"""Dense dequant GEMV (``lemoq_gemv_w8``, ``lemoq_gemv_q``) and the multi-token
linears on the matrix cores (``lemoq_gemm_w8``, ``lemoq_gemm_f16``).

Replaces ``dequant_gemm_fused`` of the reference
(``src/lemoq/kernels/_dequant_triton.py:155-293``) for every weight format it
takes: 8-bit symmetric (int8) and asymmetric (uint8 + zero point), 4-bit
symmetric and asymmetric (two codes per byte), and MXFP4 (E2M1 codes + E8M0
byte scales per 32).  Same contract: ``y = x @ dequant(qweight).T`` with fp32
dequantisation and accumulation and a single rounding to ``out_dtype`` (fp32
by default), contiguous inputs required, the same argument checks (and
exception types) before anything runs.  fp16 activations (the decode path's
type): the 8-bit symmetric branch with fp16 scales runs the decode step's GEMV,
the others ``lemoq_gemv_q``.  fp32 activations run ``lemoq_gemv_q_x32`` for
every format (fp32 products); other activation dtypes raise
``NotImplementedError``.
"""

from __future__ import annotations

from typing import Any

from lemoq import _hip

__all__ = ["DEQUANT_GEMM_CONFIGS", "dequant_gemm_fused", "dequant_gemm_separate", "linear_f16",
           "fused_available", "unavailable_reason", "warm"]

# The HIP kernel's tiling is chosen inside the library from N (rows per wave)
# and K (1 KB chunks per row); no tunables are exposed.  Kept for call-site
# compatibility with the reference's `config=` argument.
DEQUANT_GEMM_CONFIGS: dict[str, dict[str, int]] = {"dequant_gemm": {}}

MAX_PADDED_K = 8192


def unavailable_reason() -> str | None:
    """Why ``fused_available()`` is False, or None when it is True."""
    return _hip.unavailable_reason()


def fused_available() -> bool:
    """True when the HIP library is built and a ROCm device is visible (never raises)."""
    try:
        import torch  # noqa: PLC0415

        return _hip.library_available() and bool(torch.cuda.is_available())
    except Exception:  # noqa: BLE001
        return False


def _check_format(qweight: Any, scale: Any, zero: Any, group_size: int, bits: int | None, symmetric: bool,
                  mxfp4: bool) -> tuple[int, int, int]:
    """The reference's argument rules (``_dequant_triton.py:200-249``); returns
    (bits, padded_in, format id)."""
    import torch  # noqa: PLC0415

    from lemoq.quant.formats import format_id  # noqa: PLC0415

    if qweight.dim() != 2:
        raise ValueError("qweight must be 2-D (N, P), got %r" % (tuple(qweight.shape),))
    if scale.dim() != 2:
        raise ValueError("scale must be 2-D (N, n_groups), got %r" % (tuple(scale.shape),))
    N, packed_in = int(qweight.shape[0]), int(qweight.shape[1])
    n_groups = int(scale.shape[1])
    if int(scale.shape[0]) != N:
        raise ValueError("scale has %d rows, qweight has %d" % (int(scale.shape[0]), N))
    if bits is None:
        bits = 4 if qweight.dtype == torch.uint8 else 8
    bits = int(bits)
    if bits not in (4, 8):
        raise NotImplementedError("fused dequant-GEMM implements 4/8-bit, got %d" % bits)
    if mxfp4:
        if bits != 4:
            raise ValueError("mxfp4 is 4-bit E2M1 only, got bits=%r" % bits)
        if int(group_size) != 32:
            raise ValueError("the mxfp4 block is fixed at 32 (OCP MX), got group_size=%d" % int(group_size))
        if scale.dtype != torch.uint8:
            raise ValueError("mxfp4 scales must be uint8 E8M0 bytes, got %s" % scale.dtype)
        if not symmetric or zero is not None:
            raise ValueError("mxfp4 has no zero point (E2M1 carries its sign): symmetric=True and zero=None")
    padded_in = n_groups * int(group_size)
    expect_packed = padded_in if bits == 8 else padded_in // 2
    if packed_in != expect_packed:
        raise ValueError("qweight width %d != %d implied by n_groups * group_size (and bits)"
                         % (packed_in, expect_packed))
    if not symmetric and zero is None:
        raise ValueError("asymmetric quantisation needs a zero point")
    if bits == 4 and int(group_size) % 2 != 0:
        raise ValueError("4-bit needs an even group_size, got %d" % int(group_size))
    expected = torch.uint8 if (bits == 4 or not symmetric) else torch.int8
    if qweight.dtype != expected:
        raise ValueError("%d-bit qweight must be %s, got %s" % (bits, expected, qweight.dtype))
    if not mxfp4 and scale.dtype not in (torch.float16, torch.float32):
        raise ValueError("scale must be fp16 or fp32, got %s" % scale.dtype)
    if zero is not None and tuple(zero.shape) != tuple(scale.shape):
        raise ValueError("zero must have the shape of scale, got %r" % (tuple(zero.shape),))
    for name, tensor in (("qweight", qweight), ("scale", scale), ("zero", zero)):
        if tensor is not None and not tensor.is_contiguous():
            raise ValueError("%s must be contiguous" % name)
    step = 16 if bits == 8 else 32
    if int(group_size) % step != 0 or padded_in > MAX_PADDED_K:
        raise NotImplementedError(
            "the HIP GEMV needs group_size %% %d == 0 and padded_in <= %d (got group %d, padded %d)"
            % (step, MAX_PADDED_K, int(group_size), padded_in))
    return bits, padded_in, format_id(bits, symmetric, mxfp4)


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
    """``y (M, N) = x (M, K) @ dequant(qweight (N, P), scale (N, n_groups), zero).T``.

    x fp16 (``lemoq_gemv_w8`` / ``lemoq_gemv_q``: exact fp16 codes, fp16 x fp16
    products in fp32) or fp32 (``lemoq_gemv_q_x32``: fp32 products), fp32
    accumulation either way; the reference's ``_dequant_gemm_kernel``
    (``_dequant_triton.py:313-463``) in another fp32 summation order."""
    import torch  # noqa: PLC0415

    from lemoq.quant.formats import QFMT_W8, scale_zero_args  # noqa: PLC0415

    del config
    if x.dim() != 2:
        raise ValueError("x must be 2-D (M, K), got %r" % (tuple(x.shape),))
    bits, padded_in, fmt = _check_format(qweight, scale, zero, group_size, bits, symmetric, mxfp4)
    M, K = int(x.shape[0]), int(x.shape[1])
    N = int(qweight.shape[0])
    if K > padded_in:
        raise ValueError("K=%d exceeds padded_in=%d" % (K, padded_in))
    if x.dtype not in (torch.float16, torch.float32):
        raise NotImplementedError("x must be fp16 or fp32, got %s" % x.dtype)
    if not x.is_contiguous():
        raise ValueError("x must be contiguous")
    if out_dtype is None:
        out_dtype = torch.float32
    if out_dtype not in (torch.float32, torch.float16):
        raise NotImplementedError("out_dtype must be fp32 or fp16, got %s" % out_dtype)
    zero_arg = None if symmetric else zero
    scale_arg, zero_arg, s32 = scale_zero_args(scale, zero_arg)
    _hip.require_rocm(x, qweight, scale_arg, what="dequant_gemm_fused")
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    if M == 0 or N == 0:
        return y
    y16 = 1 if out_dtype == torch.float16 else 0
    st = _hip.stream_of(x.device)
    if x.dtype == torch.float32:
        _hip.call("lemoq_gemv_q_x32", _hip.ptr(x), M, K, _hip.ptr(qweight), fmt, _hip.ptr(scale_arg),
                  _hip.ptr(zero_arg) if zero_arg is not None else None, s32, N, padded_in, int(group_size),
                  _hip.ptr(y), y16, st)
    elif fmt == QFMT_W8 and not s32:
        _hip.call("lemoq_gemv_w8", _hip.ptr(x), M, K, _hip.ptr(qweight), _hip.ptr(scale_arg), N, padded_in,
                  int(group_size), _hip.ptr(y), y16, st)
    else:
        _hip.call("lemoq_gemv_q", _hip.ptr(x), M, K, _hip.ptr(qweight), fmt, _hip.ptr(scale_arg),
                  _hip.ptr(zero_arg) if zero_arg is not None else None, s32, N, padded_in, int(group_size),
                  _hip.ptr(y), y16, st)
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
    mxfp4: bool = False,
) -> Any:
    """``y (M, N) = fp16(x @ fp16(dequant(qweight)).T)`` on the matrix cores.

    The numerics of the reference's multi-token ``QuantLinear`` arm
    (``dequantized_weight(dtype=fp16)`` then ``F.linear``,
    ``src/lemoq/quant/linear.py:365-395,471-480``) without materialising the
    weight: each code is dequantised to ``fp16(code * scale)`` in registers,
    products accumulate in fp32, the output is rounded to fp16 once.  With
    ``residual`` (M, N) fp16, ``y = fp16(y + residual)``.  K must equal the
    padded width (a multiple of 64 and of ``group_size``).  The other weight
    formats (4-bit, asymmetric, MXFP4, fp32 scales) dequantise the weight to
    fp16 first (``lemoq_dequant_q``, the reference arm's materialised weight)
    and run the fp16 GEMM; they take no residual.
    """
    import torch  # noqa: PLC0415

    if x.dtype == torch.float32:  # the fp32 arm: F.linear on the fp32 dequantised weight
        return _separate_f32(x, qweight, scale, zero, group_size=group_size, bits=bits, symmetric=symmetric,
                             residual=residual, mxfp4=mxfp4)
    if mxfp4 or bits != 8 or not symmetric or zero is not None or scale.dtype != torch.float16:
        return _separate_dense(x, qweight, scale, zero, group_size=group_size, bits=bits, symmetric=symmetric,
                               residual=residual, mxfp4=mxfp4)
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


def _separate_f32(x: Any, qweight: Any, scale: Any, zero: Any, *, group_size: int, bits: int, symmetric: bool,
                  residual: Any, mxfp4: bool) -> Any:
    """Separate arm on fp32 activations: the reference's ``dequantized_weight(dtype=
    fp32)`` then ``F.linear`` in fp32 (``src/lemoq/quant/linear.py:365-395,480``).
    The fp32 weight is ``code * scale`` exactly as the fused arm forms it, so
    the fp32-activation GEMV over the M rows (``lemoq_gemv_q_x32``) computes
    the same products, accumulated in fp32 in another order; fp32 output."""
    import torch  # noqa: PLC0415

    if residual is not None:
        raise NotImplementedError("the fp32 arm takes no residual")
    bits, padded_in, _ = _check_format(qweight, scale, zero, group_size, bits, symmetric, mxfp4)
    if x.dim() != 2 or int(x.shape[1]) > padded_in:
        raise ValueError("dequant_gemm_separate: x must be (M, K <= %d), got %r" % (padded_in, tuple(x.shape)))
    return dequant_gemm_fused(x, qweight, scale, zero, group_size=group_size, bits=bits, symmetric=symmetric,
                              out_dtype=torch.float32, mxfp4=mxfp4)


def _separate_dense(x: Any, qweight: Any, scale: Any, zero: Any, *, group_size: int, bits: int, symmetric: bool,
                    residual: Any, mxfp4: bool) -> Any:
    """Separate arm for the formats the w8 matrix-core GEMM does not read:
    fp16 ``dequantized_weight`` (``src/lemoq/quant/linear.py:365-395``), then
    ``F.linear`` in fp16 with fp32 accumulation (``lemoq_gemm_f16``)."""
    from lemoq.quant.formats import dequantize  # noqa: PLC0415

    import torch  # noqa: PLC0415

    if residual is not None:
        raise NotImplementedError("the dequantise-then-GEMM arm takes no residual")
    bits, padded_in, fmt = _check_format(qweight, scale, zero, group_size, bits, symmetric, mxfp4)
    if padded_in % 64 != 0:
        raise NotImplementedError("the fp16 GEMM needs padded_in % 64 == 0, got %d" % padded_in)
    _check_rows(x, padded_in, "dequant_gemm_separate")
    w = dequantize(qweight, scale, None if symmetric else zero, fmt=fmt, group_size=group_size, k_out=padded_in,
                   dtype=torch.float16)
    return linear_f16(x, w)


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
