"""``QuantLinear`` over every weight format of the dense dequant operator,
forward through the HIP kernels.

Replaces the reference's ``QuantLinear`` (``src/lemoq/quant/linear.py:245-488``)
and its scheme table (``:76-110``, ``SchemeSpec`` ``:140-206``):

- ``w8a16``: 8-bit weights, fp16 activations (the decode path's format);
- ``w8a8``: 8-bit weights, activations fake-quantised per token to int8 before
  the linear (``_fake_quant_activation``, ``:398-414``; ``lemoq_fake_quant_rows``);
- ``w4a16``: 4-bit weights, two codes per byte;
- ``mxfp4``: E2M1 codes with an E8M0 scale per 32 (group forced to 32);
- ``fp16``: not quantised (no ``QuantLinear`` is built for it).

Buffers as the reference stores them: ``packed`` (int8 for 8-bit symmetric,
uint8 otherwise, two codes per byte at 4 bits), ``scale`` fp16 (uint8 E8M0 for
MXFP4), ``zero`` fp16 for asymmetric schemes else ``None``, ``bias``.

``forward`` dispatches as the reference does (``_fused_fallback_reason``,
``:420-444``): in ``dequant="fused"`` mode (the default here, the decode path)
one token takes the fused dequant-GEMV (fp32 dequantisation, one rounding);
several tokens, or ``dequant="separate"``, take the separate arm's numerics
(fp16 ``dequantized_weight`` + ``F.linear`` with fp32 accumulation,
``:365-395,471-480``) on the matrix cores: the 8-bit symmetric GEMM dequantises
in registers, the other formats materialise the fp16 weight first.
Quantisation runs on the device (``lemoq.quant.rtn``, ``lemoq.quant.mxfp4``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch
from torch import nn

__all__ = ["DEQUANT_MODES", "QuantLinear", "SchemeSpec", "parse_scheme"]

# scheme name -> (weight bits, activation bits or None)
_SCHEMES = {
    "w8a8": (8, 8),
    "w8a16": (8, None),
    "w4a16": (4, None),
    "mxfp4": (4, None),
    "fp16": (None, None),
}

DEQUANT_MODES: tuple[str, ...] = ("separate", "fused")


def parse_scheme(name: str) -> tuple[int | None, int | None]:
    """``"w4a16"`` -> ``(4, None)``; ``"w8a8"`` -> ``(8, 8)``; ``"fp16"`` -> ``(None, None)``."""
    key = str(name).lower()
    if key not in _SCHEMES:
        raise ValueError("unknown scheme %r; implemented: %s" % (name, sorted(_SCHEMES)))
    return _SCHEMES[key]


@dataclass(frozen=True)
class SchemeSpec:
    """One quantisation configuration (the reference's fields that the operator reads)."""

    name: str
    weight_bits: int | None
    act_bits: int | None
    group_size: int | None
    targets: tuple[str, ...] = ("attention", "experts", "router")
    keep_lm_head_fp16: bool = True
    symmetric: bool = True
    scheme: str = "rtn"
    dequant: str = "fused"

    def __post_init__(self) -> None:
        if str(self.dequant) not in DEQUANT_MODES:
            raise ValueError("unknown dequant mode %r; implemented: %s" % (self.dequant, list(DEQUANT_MODES)))
        if self.scheme != "rtn":
            raise NotImplementedError("only RTN quantisation is built (GPTQ needs calibration data)")

    @classmethod
    def from_flags(cls, name: str, group_size: int, *, targets: tuple[str, ...] | None = None,
                   keep_lm_head_fp16: bool = True, dequant: str = "fused", symmetric: bool = True) -> "SchemeSpec":
        bits, act = parse_scheme(name)
        if name == "mxfp4":
            group_size = 32  # the OCP MX block
        return cls(name=name, weight_bits=bits, act_bits=act, group_size=group_size,
                   targets=targets or ("attention", "experts", "router"), keep_lm_head_fp16=keep_lm_head_fp16,
                   symmetric=symmetric, dequant=str(dequant))

    @property
    def enabled(self) -> bool:
        return self.weight_bits is not None


class QuantLinear(nn.Module):
    def __init__(self, weight: Any, *, group_size: int = 128, bias: Any = None, name: str = "",
                 scheme: str = "w8a16", symmetric: bool = True, dequant: str = "fused") -> None:
        super().__init__()
        bits, act = parse_scheme(scheme)
        if bits is None:
            raise ValueError("scheme %r is not quantised: keep an nn.Linear" % scheme)
        if dequant not in DEQUANT_MODES:
            raise ValueError("unknown dequant mode %r" % dequant)
        if weight.dim() != 2:
            raise ValueError("weight must be 2-D (out, in)")
        self.name = name
        self.scheme = str(scheme)
        self.in_features = int(weight.shape[1])
        self.out_features = int(weight.shape[0])
        self.weight_bits = int(bits)
        self.act_bits = act
        self.dequant_mode = str(dequant)
        if scheme == "mxfp4":
            from lemoq.quant.mxfp4 import quantize_mxfp4  # noqa: PLC0415

            if not symmetric:
                raise ValueError("mxfp4 has no zero point")
            qm = quantize_mxfp4(weight.detach(), block=32)
            self.symmetric = True
            self.group_size = 32
            self.padded_in = int(qm["padded_in"])
            self.n_groups = int(qm["scales"].shape[1])
            self.register_buffer("packed", qm["codes_packed"].contiguous(), persistent=True)
            self.register_buffer("scale", qm["scales"].contiguous(), persistent=True)
            self.register_buffer("zero", None)
        else:
            from lemoq.quant import rtn  # noqa: PLC0415

            q = rtn.quantize_rtn(weight.detach(), bits=self.weight_bits, group_size=group_size, symmetric=symmetric)
            self.symmetric = bool(symmetric)
            self.group_size = int(group_size)
            self.padded_in = int(q["padded_in"])
            self.n_groups = int(q["n_groups"])
            self.register_buffer("packed", q["packed"].contiguous(), persistent=True)
            self.register_buffer("scale", q["scale_f16"].contiguous(), persistent=True)
            self.register_buffer("zero", None if symmetric else q["zero_f16"].contiguous())
        self.register_buffer("bias", bias.detach().clone() if bias is not None else None, persistent=True)

    @classmethod
    def from_linear(cls, linear: Any, spec: SchemeSpec, *, name: str = "") -> "QuantLinear":
        """The reference's constructor form: an ``nn.Linear`` and a ``SchemeSpec``."""
        if not spec.enabled:
            raise ValueError("SchemeSpec.weight_bits is None: keep the nn.Linear")
        return cls(linear.weight.detach(), group_size=int(spec.group_size or 128),
                   bias=linear.bias.detach() if linear.bias is not None else None, name=name, scheme=spec.name,
                   symmetric=spec.symmetric, dequant=spec.dequant)

    @classmethod
    def from_packed(cls, packed: Any, scale: Any, *, in_features: int, group_size: int, bias: Any = None,
                    name: str = "", zero: Any = None, scheme: str = "w8a16", symmetric: bool = True,
                    dequant: str = "fused") -> "QuantLinear":
        """Wrap already-quantized buffers (e.g. a checkpoint) without re-quantizing."""
        bits, act = parse_scheme(scheme)
        if bits is None:
            raise ValueError("scheme %r is not quantised" % scheme)
        obj = cls.__new__(cls)
        nn.Module.__init__(obj)
        obj.name = name
        obj.scheme = str(scheme)
        obj.in_features = int(in_features)
        obj.out_features = int(packed.shape[0])
        obj.weight_bits = int(bits)
        obj.act_bits = act
        obj.symmetric = bool(symmetric)
        obj.dequant_mode = str(dequant)
        obj.group_size = 32 if scheme == "mxfp4" else int(group_size)
        obj.n_groups = int(scale.shape[1])
        obj.padded_in = obj.n_groups * obj.group_size
        width = obj.padded_in if bits == 8 else obj.padded_in // 2
        if int(packed.shape[1]) != width:
            raise ValueError("packed width %d != %d implied by scale groups x group_size"
                             % (int(packed.shape[1]), width))
        if not symmetric and zero is None:
            raise ValueError("an asymmetric scheme needs its zero points")
        obj.register_buffer("packed", packed.contiguous(), persistent=True)
        obj.register_buffer("scale", scale.contiguous(), persistent=True)
        obj.register_buffer("zero", None if symmetric else zero.contiguous())
        obj.register_buffer("bias", bias, persistent=True)
        return obj

    @property
    def mxfp4(self) -> bool:
        return self.scheme == "mxfp4"

    def dequantized_weight(self, dtype: Any = None) -> Any:
        """(out, in) weight: fp32 ``code * scale`` / ``(code - zero) * scale`` /
        ``e2m1 * 2^(X-127)``, rounded once to ``dtype`` when given
        (``src/lemoq/quant/linear.py:365-395``)."""
        from lemoq.quant.formats import dequantize, format_id  # noqa: PLC0415

        out = dtype if dtype in (torch.float16, torch.float32) else torch.float32
        w = dequantize(self.packed, self.scale, self.zero, fmt=format_id(self.weight_bits, self.symmetric, self.mxfp4),
                       group_size=self.group_size, k_out=self.in_features, dtype=out)
        return w if dtype is None or dtype == out else w.to(dtype)

    def _fake_quant_activation(self, x: Any) -> Any:
        """Per-token symmetric int8 fake quantisation (w8a8); identity otherwise."""
        from lemoq import _hip  # noqa: PLC0415

        if self.act_bits is None:
            return x
        if x.dtype != torch.float16:
            raise NotImplementedError("w8a8 activations must be fp16, got %s" % x.dtype)
        _hip.require_rocm(x, what="QuantLinear w8a8")
        flat = x.reshape(-1, int(x.shape[-1])).contiguous()
        y = torch.empty_like(flat)
        _hip.call("lemoq_fake_quant_rows", _hip.ptr(flat), int(flat.shape[0]), int(flat.shape[1]), _hip.ptr(y),
                  _hip.stream_of(x.device))
        return y.reshape(x.shape)

    def forward(self, x: Any) -> Any:
        from lemoq.kernels.dequant_gemm import dequant_gemm_fused, dequant_gemm_separate  # noqa: PLC0415

        if x.shape[-1] != self.in_features:
            raise ValueError("input width %d != in_features %d" % (int(x.shape[-1]), self.in_features))
        xq = self._fake_quant_activation(x)
        flat = xq.reshape(-1, self.in_features)
        flat = flat if flat.is_contiguous() else flat.contiguous()
        zero = None if self.symmetric else self.zero
        if int(flat.shape[0]) == 1 and self.dequant_mode == "fused":
            y = dequant_gemm_fused(flat, self.packed, self.scale, zero, group_size=self.group_size,
                                   bits=self.weight_bits, symmetric=self.symmetric, out_dtype=x.dtype,
                                   mxfp4=self.mxfp4)
        else:
            xs = flat
            if self.padded_in != self.in_features:  # padded columns: zero inputs add nothing
                xs = torch.nn.functional.pad(xs, (0, self.padded_in - self.in_features))
            y = dequant_gemm_separate(xs, self.packed, self.scale, zero, group_size=self.group_size,
                                      bits=self.weight_bits, symmetric=self.symmetric, mxfp4=self.mxfp4)
            y = y if x.dtype == y.dtype else y.to(x.dtype)
        y = y.reshape(*x.shape[:-1], self.out_features)
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        return y

    def extra_repr(self) -> str:
        return "%d->%d %s%s group=%d" % (self.in_features, self.out_features, self.scheme,
                                        "" if self.symmetric else " asym", self.group_size)
