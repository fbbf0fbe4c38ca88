"""Packed q/k/v projection: one w8 GEMV launch for the three attention inputs.

Mirrors ``PackedQKV`` of the reference (``src/lemoq/kernels/packed_qkv.py:68-103``):
the three symmetric w8 ``QuantLinear`` weights are concatenated along the output
dimension and projected with one ``dequant_gemm_fused`` call.  The layout is
row-local (each output row reads only its own codes and scales), so every
packed row equals the single-projection row bit for bit.
``pack_qkv(q_proj, k_proj, v_proj)`` builds one; ``install_packed_qkv(model)``
attaches one to every attention module of a model (a module with ``q_proj``,
``k_proj`` and ``v_proj``, as ``_lemoq_packed_qkv``, the reference's attribute),
``packed_qkv_installed`` / ``remove_packed_qkv`` count and drop them
(``:104-170``), and ``packed_qkv_enabled`` / ``packed_qkv_applicable`` are the
reference's switch and preconditions (``:40-58``).  This build's own decode step
packs q|k|v in its weights (``OlmoeW8Weights.qkv_codes``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

__all__ = ["PackedQKV", "install_packed_qkv", "pack_qkv", "packed_qkv_applicable", "packed_qkv_enabled",
           "packed_qkv_installed", "remove_packed_qkv"]

_ATTR = "_lemoq_packed_qkv"


def packed_qkv_enabled() -> bool:
    """The ``packed_qkv`` fusion switch (``LEMOQ_PACKED_QKV``)."""
    from lemoq.kernels.fusion_switches import fusion_enabled  # noqa: PLC0415

    return fusion_enabled("packed_qkv")


def packed_qkv_applicable(attn: Any, quantized: bool) -> bool:
    """The two preconditions: the attention kernel cell and quantised projections
    (fp16 q/k/v are plain linears: nothing to pack; not applicable means no-op)."""
    return str(attn) == "kernel" and bool(quantized)


def _attention_modules(model: Any) -> list:
    return [m for m in model.modules() if all(hasattr(m, n) for n in ("q_proj", "k_proj", "v_proj"))]


def install_packed_qkv(model: Any) -> int:
    """Attach a ``PackedQKV`` to every attention module of ``model``; returns how
    many.  Run after quantisation and before graph capture (it allocates).
    Raises when no module has q/k/v projections, or one is not packable."""
    mods = _attention_modules(model)
    if not mods:
        raise RuntimeError("no attention module (q_proj, k_proj, v_proj) found")
    for m in mods:
        setattr(m, _ATTR, pack_qkv(m.q_proj, m.k_proj, m.v_proj))
    return len(mods)


def packed_qkv_installed(model: Any) -> int:
    """How many attention modules carry a packed q/k/v state."""
    return sum(1 for m in _attention_modules(model) if getattr(m, _ATTR, None) is not None)


def remove_packed_qkv(model: Any) -> int:
    """Drop the packed states (A/B arms in one process); returns how many."""
    n = 0
    for m in _attention_modules(model):
        if getattr(m, _ATTR, None) is not None:
            delattr(m, _ATTR)
            n += 1
    return n


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
