"""Packed q/k/v projection: one w8 GEMV launch for the three attention inputs.

Mirrors ``PackedQKV`` of the reference (``src/lemoq/kernels/packed_qkv.py:68-103``):
the three symmetric w8 ``QuantLinear`` weights are concatenated along the output
dimension and projected with one ``dequant_gemm_fused`` call.  The layout is
row-local (each output row reads only its own codes and scales), so every
packed row equals the single-projection row bit for bit.
``pack_qkv(q_proj, k_proj, v_proj)`` replaces ``install_packed_qkv`` (which
patched HF modules; this build owns its decode module).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

__all__ = ["PackedQKV", "pack_qkv"]


@dataclass
class PackedQKV:
    packed: Any
    scale: Any
    in_features: int
    out_features: int
    group_size: int

    def _packed_rows(self, x: Any) -> Any:
        """The one GEMV/GEMM launch: ``(M, in)`` rows -> ``(M, 3*out)``, q | k | v."""
        from lemoq.kernels.dequant_gemm import dequant_gemm_fused  # noqa: PLC0415

        rows = x.reshape(-1, self.in_features).contiguous()
        return dequant_gemm_fused(rows, self.packed, self.scale, None, group_size=self.group_size,
                                  bits=8, symmetric=True, out_dtype=x.dtype)

    def project(self, x: Any) -> tuple[Any, Any, Any]:
        """``(..., in)`` -> q, k, v of shape ``(..., out)`` each: views of one
        packed output, no copies."""
        y = self._packed_rows(x).view(*x.shape[:-1], 3, self.out_features)
        return tuple(y.unbind(-2))

    def combined(self, x: Any) -> Any:
        """The packed ``(..., 3*out)`` output itself."""
        return self._packed_rows(x).view(*x.shape[:-1], 3 * self.out_features)


def pack_qkv(q: Any, k: Any, v: Any) -> PackedQKV:
    """Concatenate three w8 ``QuantLinear`` projections (same shapes) into one."""
    import torch  # noqa: PLC0415

    from lemoq.quant.linear import QuantLinear  # noqa: PLC0415

    for role, m in (("q_proj", q), ("k_proj", k), ("v_proj", v)):
        if not isinstance(m, QuantLinear):
            raise ValueError("packed q/k/v needs quantized %s, got %s" % (role, type(m).__name__))
        if int(m.weight_bits) != 8:
            raise NotImplementedError("packed q/k/v supports w8 only (%s)" % role)
        if m.zero is not None:
            raise NotImplementedError("packed q/k/v supports symmetric weights only (%s)" % role)
        if getattr(m, "act_bits", None) is not None:
            raise NotImplementedError("packed q/k/v supports fp16 activations only (%s is w8a8)" % role)
        if m.bias is not None:
            raise NotImplementedError("packed q/k/v does not support biased projections (%s)" % role)
    shape = {
        (int(m.in_features), int(m.out_features), int(m.group_size), int(m.padded_in), int(m.n_groups))
        for m in (q, k, v)
    }
    if len(shape) != 1:
        raise ValueError("q/k/v need identical (in, out, group, padded_in, n_groups), got %r" % (sorted(shape),))
    return PackedQKV(
        packed=torch.cat((q.packed, k.packed, v.packed), dim=0).contiguous(),
        scale=torch.cat((q.scale, k.scale, v.scale), dim=0).contiguous(),
        in_features=int(q.in_features),
        out_features=int(q.out_features),
        group_size=int(q.group_size),
    )
