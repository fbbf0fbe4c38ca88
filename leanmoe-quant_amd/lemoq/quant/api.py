"""The stable quantisation entry points of ``lemoq.quant`` (the reference's
``src/lemoq/quant/api.py:1-191``): ``quantize_linear`` -> ``QuantizedLinear`` and
``dequantize_reference``, plus ``REMEDIATION_LADDER``, the ordered list of the
legal ways to recover accuracy when a format misses the quality gate.

Only RTN is built (``lemoq.quant.rtn``, on the device); GPTQ needs calibration
data and is refused with ``NotImplementedError`` before anything is computed.
``dequantize_reference`` is the fp32 dequantisation every kernel is checked
against (``lemoq_dequant_q``).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

__all__ = ["QuantizedLinear", "REMEDIATION_LADDER", "dequantize_reference", "quantize_linear"]

# Escalation order when a quantised model misses the KL / top-1 gate; every
# step has to pass the gate again.  Which of them this build has: 1 (RTN, the
# device quantiser) and 5 (SchemeSpec.targets / keep_lm_head_fp16 choose what
# is quantised); 2-4 need calibration data.
REMEDIATION_LADDER: tuple[dict[str, str], ...] = (
    {"step": "1_rtn", "method": "per-group round-to-nearest", "needs_calibration": "no",
     "built_here": "yes (lemoq.quant.rtn)"},
    {"step": "2_gptq", "method": "layer-wise reconstruction against calibration activations",
     "needs_calibration": "yes", "built_here": "no"},
    {"step": "3_awq", "method": "activation-aware per-channel scaling", "needs_calibration": "yes",
     "built_here": "no"},
    {"step": "4_mixed_bits", "method": "higher bit width for the sensitive layers or experts",
     "needs_calibration": "yes", "built_here": "no"},
    {"step": "5_selective", "method": "quantise the experts only, keep lm_head and attention fp16",
     "needs_calibration": "no", "built_here": "yes (SchemeSpec.targets, keep_lm_head_fp16)"},
)


@dataclass
class QuantizedLinear:
    """A quantised 2-D weight and what dequantising it needs.  ``codes`` are the
    unpacked codes (int8 for 8-bit symmetric, uint8 otherwise, width
    ``in_features``); ``meta`` holds ``n_groups``, ``padded_in``, ``device`` and the
    packed storage (``packed``) the operators read."""

    codes: Any
    scale: Any
    zero: Any
    bits: int
    group_size: int
    symmetric: bool
    scheme: str
    shape: tuple[int, int]
    meta: dict[str, Any] = field(default_factory=dict)

    @property
    def n_params(self) -> int:
        return self.shape[0] * self.shape[1]


def quantize_linear(weight: Any, *, bits: int = 4, group_size: int = 128, scheme: str = "rtn",
                    symmetric: bool = True, calibration: Any = None, block_size: int = 128, damp: float = 0.01,
                    min_samples: int = 256) -> QuantizedLinear:
    """Quantise a 2-D device weight with ``scheme`` (``"rtn"``).  The GPTQ
    arguments (``calibration``, ``block_size``, ``damp``, ``min_samples``) are
    accepted for call-site compatibility and refused with the scheme."""
    del block_size, damp, min_samples
    if scheme not in ("rtn", "gptq"):
        raise NotImplementedError("scheme=%r is not implemented; 'rtn' is (see REMEDIATION_LADDER)" % (scheme,))
    if scheme == "gptq":
        raise NotImplementedError("GPTQ needs calibration data and is not built here; use scheme='rtn'")
    if calibration is not None:
        raise ValueError("RTN does not consume calibration data")
    from lemoq.quant import rtn  # noqa: PLC0415

    q = rtn.quantize_rtn(weight, bits=bits, group_size=group_size, symmetric=symmetric)
    return QuantizedLinear(codes=q["codes"], scale=q["scale"], zero=q["zero"], bits=int(bits),
                           group_size=int(group_size), symmetric=bool(symmetric), scheme=scheme, shape=q["shape"],
                           meta={"n_groups": q["n_groups"], "padded_in": q["padded_in"], "device": q["device"],
                                 "packed": q["packed"]})


def dequantize_reference(qlinear: QuantizedLinear) -> Any:
    """fp32 ``codes * scale`` (``(codes - zero) * scale`` asymmetric), shape
    ``qlinear.shape``: the dequantisation the kernels are held to."""
    import torch  # noqa: PLC0415

    from lemoq.quant import rtn  # noqa: PLC0415
    from lemoq.quant.pack import pack_4bit  # noqa: PLC0415

    packed = qlinear.meta.get("packed")
    if packed is None:  # built from unpacked codes: pad to the group grid, pack at 4 bits
        rows, cols = qlinear.shape
        padded = torch.zeros((rows, int(qlinear.meta["padded_in"])), dtype=qlinear.codes.dtype,
                             device=qlinear.codes.device)
        padded[:, :cols] = qlinear.codes
        packed = pack_4bit(padded) if qlinear.bits == 4 else padded
    q = {"packed": packed, "scale": qlinear.scale, "zero": qlinear.zero, "bits": qlinear.bits,
         "group_size": qlinear.group_size, "symmetric": qlinear.symmetric, "shape": qlinear.shape}
    return rtn.dequantize_rtn(q)
