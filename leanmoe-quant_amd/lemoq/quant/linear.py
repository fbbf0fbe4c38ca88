"""``QuantLinear`` for w8 symmetric per-group weights, forward through the HIP GEMV.

Replaces the part of the reference's ``QuantLinear`` (``src/lemoq/quant/linear.py:245-488``)
that the decode path uses: buffers ``packed`` int8 (out, padded_in), ``scale``
fp16 (out, n_groups), ``zero=None``, ``bias`` (optional).  ``forward``
dispatches as the reference does (``_fused_fallback_reason``, ``:420-444``):
one token takes the fused dequant-GEMV (``_fused_forward``, ``:446-469``;
fp32 dequantisation, one rounding), several tokens take the numerics of the
"separate" arm (``dequantized_weight`` + ``F.linear``, ``:365-395,471-480``:
fp16 weight, fp32 accumulation) on the matrix-core GEMM, which dequantises in
registers instead of materialising the fp16 weight.  Quantisation runs on the
device (``lemoq.quant.rtn``).
"""

from __future__ import annotations

from typing import Any

import torch
from torch import nn

__all__ = ["QuantLinear"]


class QuantLinear(nn.Module):
    def __init__(self, weight: Any, *, group_size: int = 128, bias: Any = None, name: str = "") -> None:
        super().__init__()
        from lemoq.quant import rtn  # noqa: PLC0415

        if weight.dim() != 2:
            raise ValueError("weight must be 2-D (out, in)")
        q = rtn.quantize_rtn(weight.detach(), bits=8, group_size=group_size, symmetric=True)
        self.name = name
        self.in_features = int(weight.shape[1])
        self.out_features = int(weight.shape[0])
        self.weight_bits = 8
        self.group_size = int(group_size)
        self.padded_in = int(q["padded_in"])
        self.n_groups = int(q["n_groups"])
        self.register_buffer("packed", q["codes_padded"].contiguous(), persistent=True)
        self.register_buffer("scale", q["scale_f16"].contiguous(), persistent=True)
        self.register_buffer("zero", None)
        self.register_buffer("bias", bias.detach().clone() if bias is not None else None, persistent=True)

    @classmethod
    def from_packed(cls, packed: Any, scale: Any, *, in_features: int, group_size: int, bias: Any = None,
                    name: str = "") -> "QuantLinear":
        """Wrap already-quantized buffers (e.g. a checkpoint) without re-quantizing."""
        obj = cls.__new__(cls)
        nn.Module.__init__(obj)
        obj.name = name
        obj.in_features = int(in_features)
        obj.out_features = int(packed.shape[0])
        obj.weight_bits = 8
        obj.group_size = int(group_size)
        obj.padded_in = int(packed.shape[1])
        obj.n_groups = int(scale.shape[1])
        if obj.n_groups * obj.group_size != obj.padded_in:
            raise ValueError("scale groups x group_size != packed width")
        obj.register_buffer("packed", packed.contiguous(), persistent=True)
        obj.register_buffer("scale", scale.contiguous(), persistent=True)
        obj.register_buffer("zero", None)
        obj.register_buffer("bias", bias, persistent=True)
        return obj

    def forward(self, x: Any) -> Any:
        from lemoq.kernels.dequant_gemm import dequant_gemm_fused, dequant_gemm_separate  # noqa: PLC0415

        if x.shape[-1] != self.in_features:
            raise ValueError("input width %d != in_features %d" % (int(x.shape[-1]), self.in_features))
        flat = x.reshape(-1, self.in_features)
        flat = flat if flat.is_contiguous() else flat.contiguous()
        if int(flat.shape[0]) == 1:
            y = dequant_gemm_fused(flat, self.packed, self.scale, None, group_size=self.group_size, bits=8,
                                   symmetric=True, out_dtype=x.dtype)
        else:
            xs = flat
            if self.padded_in != self.in_features:  # padded columns hold code 0: zero inputs add nothing
                xs = torch.nn.functional.pad(xs, (0, self.padded_in - self.in_features))
            y = dequant_gemm_separate(xs, self.packed, self.scale, None, group_size=self.group_size)
            y = y if x.dtype == y.dtype else y.to(x.dtype)
        y = y.reshape(*x.shape[:-1], self.out_features)
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        return y

    def extra_repr(self) -> str:
        return "%d->%d w8 group=%d" % (self.in_features, self.out_features, self.group_size)
