"""4-bit packing of quantised codes: two codes per byte, the even column in
the low nibble.

The reference's convention (``src/lemoq/quant/pack.py:1-63``):
``byte = (c[2j] & 0xF) | ((c[2j + 1] & 0xF) << 4)``; unpacking sign-extends
the nibbles of symmetric int4 codes (-8 .. 7) and leaves asymmetric uint4
codes (0 .. 15) and MXFP4 E2M1 codes unsigned.  These are tensor bit
operations on whatever device the tensor lives on; the HIP quantisers
(``lemoq_rtn_quantize``, ``lemoq_mxfp4_quantize``) write the packed layout
directly, and the HIP GEMV / dequantisation read it.  Byte accounting
(``packed_nbytes``, ``scale_nbytes``, ``bit_cost``) follows
``src/lemoq/quant/pack.py:66-129``.
"""

from __future__ import annotations

from typing import Any

__all__ = ["pack_4bit", "unpack_4bit", "packed_nbytes", "scale_nbytes", "bit_cost"]


def pack_4bit(codes: Any) -> Any:
    """Pack 4-bit codes (last dim even, any integer dtype) into uint8."""
    import torch  # noqa: PLC0415

    last = int(codes.shape[-1])
    if last % 2 != 0:
        raise ValueError("the last dim must be even to pack 4-bit codes, got %d" % last)
    c = codes.to(torch.int32)
    lo = (c[..., 0::2] & 0xF).to(torch.uint8)
    hi = ((c[..., 1::2] & 0xF) << 4).to(torch.uint8)
    return lo | hi


def unpack_4bit(packed: Any, *, signed: bool = True) -> Any:
    """Inverse of ``pack_4bit``: int8 -8 .. 7 when ``signed``, else uint8 0 .. 15."""
    import torch  # noqa: PLC0415

    p = packed.to(torch.int32)
    out = torch.stack((p & 0xF, (p >> 4) & 0xF), dim=-1).reshape(*packed.shape[:-1], int(packed.shape[-1]) * 2)
    if signed:
        out = torch.where(out >= 8, out - 16, out)
    return out.to(torch.int8 if signed else torch.uint8)


def packed_nbytes(n_params: int, bits: int) -> int:
    """Packed weight bytes for ``n_params`` codes at ``bits``."""
    if bits not in (4, 8):
        raise ValueError("only 4 or 8 bit")
    return n_params * bits // 8


def scale_nbytes(n_params: int, group_size: int, scale_bytes: int = 2, *, in_features: int | None = None) -> int:
    """Per-group scale bytes.  Groups run along the input dim of each output row:
    ``rows * ceil(in_features / group_size)`` with ``in_features`` given, else
    ``ceil(n_params / group_size)`` (exact only when the width divides)."""
    if group_size <= 0:
        return 0
    if in_features is None:
        n_groups = -(-n_params // group_size)
    else:
        in_features = int(in_features)
        if in_features <= 0:
            raise ValueError("in_features must be > 0, got %r" % (in_features,))
        if n_params % in_features != 0:
            raise ValueError("n_params=%d is not a multiple of in_features=%d" % (n_params, in_features))
        n_groups = (n_params // in_features) * -(-in_features // group_size)
    return n_groups * scale_bytes


def bit_cost(n_params: int, bits: int, group_size: int, scale_bytes: int = 2, *,
             in_features: int | None = None) -> dict[str, int]:
    """Total quantised footprint: packed codes plus scales."""
    p = packed_nbytes(n_params, bits)
    s = scale_nbytes(n_params, group_size, scale_bytes, in_features=in_features)
    return {"params": n_params, "packed_bytes": p, "scale_bytes": s, "total_bytes": p + s}
