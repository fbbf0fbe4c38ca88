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
one fp16 or fp32 token takes the fused dequant-GEMV (fp32 dequantisation, one
rounding); several tokens, or ``dequant="separate"``, take the separate arm's
numerics (``dequantized_weight`` in the activation's dtype + ``F.linear``,
``:365-395,471-480``): for fp16 on the matrix cores (the 8-bit symmetric GEMM
dequantises in registers, the other formats materialise the fp16 weight
first), for fp32 through the fp32-activation GEMV.  Every call is counted the
reference's way (``_counters``: fused calls, separate calls, the reason for
each fallback), and the module-level helpers read and reset the counts over a
whole model (``set_dequant_mode``, ``reset_dequant_counters``,
``dequant_activity``, ``supported_dequant_modes``, ``:113-125,529-589``).
``quantize_model`` replaces a model's ``nn.Linear`` modules by name as the
reference's does (``:592-694``).  Quantisation runs on the device
(``lemoq.quant.rtn``, ``lemoq.quant.mxfp4``); there is no CPU arm.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field
from typing import Any

import torch
from torch import nn

__all__ = ["DEQUANT_MODES", "QuantLinear", "QuantizeReport", "SchemeSpec", "TARGET_RULES", "classify_linear",
           "dequant_activity", "parse_scheme", "quantize_model", "realized_bytes", "reset_dequant_counters",
           "set_dequant_mode", "supported_dequant_modes"]

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

    def to_dict(self) -> dict[str, Any]:
        """The spec as a result's ``config`` records it (the reference's keys)."""
        return {
            "scheme": self.name,
            "weight_bits": self.weight_bits,
            "act_bits": self.act_bits,
            "group_size": self.group_size,
            "targets": list(self.targets),
            "keep_lm_head_fp16": self.keep_lm_head_fp16,
            "symmetric": self.symmetric,
            "rtn_scheme": self.scheme,
            "dequant": self.dequant,
            "activation_quantization": "fake-quant (quantised, then dequantised at once; no int8 GEMM)"
            if self.act_bits is not None else None,
        }


# Which [W] term an nn.Linear belongs to, by its full module name in an HF
# OLMoE model (`model.layers.3.self_attn.q_proj`, `model.layers.0.mlp.experts.17.
# gate_proj`, `model.layers.5.mlp.gate`, `lm_head`): the reference's rules
# (src/lemoq/quant/linear.py:214-220), first match wins, no match = not quantised.
TARGET_RULES: tuple[tuple[str, str], ...] = (
    (r"^lm_head$", "lm_head"),
    (r"\.self_attn\.", "attention"),
    (r"\.experts\.\d+\.", "experts"),
    (r"\.mlp\.gate$", "router"),
    (r"\.shared_expert", "shared"),
)
_LAYER_INDEX = re.compile(r"\.layers\.(\d+)\.")


def classify_linear(module_name: str) -> str | None:
    """The target of a linear's full module name, or None (kept unquantised)."""
    return next((target for pattern, target in TARGET_RULES if re.search(pattern, module_name)), None)


def _layer_index(module_name: str) -> int | None:
    m = _LAYER_INDEX.search(module_name)
    return int(m.group(1)) if m else None


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
        self._counters = _fresh_counters()

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
        obj._counters = _fresh_counters()
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

    @property
    def fused_available(self) -> bool:
        """Whether the fused arm can run here (the HIP library and a ROCm device); never raises."""
        from lemoq.kernels.dequant_gemm import fused_available  # noqa: PLC0415

        return fused_available()

    def _fused_fallback_reason(self, x: Any) -> str | None:
        """Why this call cannot take the fused arm, as the reference words it
        (``src/lemoq/quant/linear.py:420-444``), or None.  Static host checks only,
        so a captured call always dispatches the same way."""
        import torch  # noqa: PLC0415

        if self.dequant_mode != "fused":
            return "mode_is_separate"
        if not x.is_cuda:
            return "not_cuda"
        if x.dtype not in (torch.float16, torch.float32):
            return "dtype_unsupported(%s)" % str(x.dtype).replace("torch.", "")
        if self.weight_bits not in (4, 8):
            return "bits_unsupported(%d)" % self.weight_bits
        if int(x.shape[-1]) != self.in_features:
            return "input_width_mismatch(%d!=%d)" % (int(x.shape[-1]), self.in_features)
        if int(x.numel()) // max(self.in_features, 1) != 1:
            return "multi_token"
        if not self.fused_available:
            from lemoq.kernels.dequant_gemm import unavailable_reason  # noqa: PLC0415

            return "kernel_unavailable(%s)" % (unavailable_reason() or "unknown")
        return None

    def forward(self, x: Any) -> Any:
        from lemoq.kernels.dequant_gemm import dequant_gemm_fused, dequant_gemm_separate  # noqa: PLC0415

        if x.shape[-1] != self.in_features:
            raise ValueError("input width %d != in_features %d" % (int(x.shape[-1]), self.in_features))
        xq = self._fake_quant_activation(x)
        flat = xq.reshape(-1, self.in_features)
        flat = flat if flat.is_contiguous() else flat.contiguous()
        zero = None if self.symmetric else self.zero
        reason = self._fused_fallback_reason(xq)
        if reason is None:
            y = dequant_gemm_fused(flat, self.packed, self.scale, zero, group_size=self.group_size,
                                   bits=self.weight_bits, symmetric=self.symmetric, out_dtype=x.dtype,
                                   mxfp4=self.mxfp4)
            self._counters["fused_calls"] += 1
        else:
            xs = flat
            if self.padded_in != self.in_features:  # padded columns: zero inputs add nothing
                xs = torch.nn.functional.pad(xs, (0, self.padded_in - self.in_features))
            y = dequant_gemm_separate(xs, self.packed, self.scale, zero, group_size=self.group_size,
                                      bits=self.weight_bits, symmetric=self.symmetric, mxfp4=self.mxfp4)
            y = y if x.dtype == y.dtype else y.to(x.dtype)
            # counted once the arm has run (this build has no CPU arm: a CPU input raises above)
            if reason != "mode_is_separate":
                fb = self._counters["fallbacks"]
                fb[reason] = fb.get(reason, 0) + 1
            self._counters["separate_calls"] += 1
        y = y.reshape(*x.shape[:-1], self.out_features)
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        return y

    def extra_repr(self) -> str:
        return "%d->%d %s%s group=%d" % (self.in_features, self.out_features, self.scheme,
                                        "" if self.symmetric else " asym", self.group_size)


def _fresh_counters() -> dict[str, Any]:
    return {"separate_calls": 0, "fused_calls": 0, "fallbacks": {}}


def _quant_linears(model: Any):
    return (m for m in model.modules() if isinstance(m, QuantLinear))


def supported_dequant_modes(model: Any) -> tuple[str, ...]:
    """``("separate", "fused")`` when the model's QuantLinear modules can take the
    fused arm here, else ``("separate",)`` (``src/lemoq/quant/linear.py:113-124``)."""
    first = next(_quant_linears(model), None)
    return ("separate", "fused") if first is not None and first.fused_available else ("separate",)


def set_dequant_mode(model: Any, mode: str) -> int:
    """Switch every QuantLinear of ``model`` to ``mode``; returns how many were
    switched (the arms share the packed weights, so both can alternate on one
    model instance; ``:529-545``)."""
    key = str(mode)
    if key not in DEQUANT_MODES:
        raise ValueError("unknown dequant mode %r; implemented: %s" % (mode, list(DEQUANT_MODES)))
    n = 0
    for m in _quant_linears(model):
        m.dequant_mode = key
        n += 1
    return n


def reset_dequant_counters(model: Any) -> int:
    """Zero the dispatch counts of every QuantLinear of ``model``; returns how many."""
    n = 0
    for m in _quant_linears(model):
        m._counters = _fresh_counters()
        n += 1
    return n


def dequant_activity(model: Any) -> dict[str, Any]:
    """The dispatches that actually happened, summed over the model (``:558-589``):
    ``fused_calls == 0`` with ``fallbacks`` set means the separate arm ran."""
    modes: dict[str, int] = {}
    fallbacks: dict[str, int] = {}
    n = fused = separate = 0
    for m in _quant_linears(model):
        n += 1
        modes[m.dequant_mode] = modes.get(m.dequant_mode, 0) + 1
        fused += int(m._counters["fused_calls"])
        separate += int(m._counters["separate_calls"])
        for reason, count in m._counters["fallbacks"].items():
            fallbacks[reason] = fallbacks.get(reason, 0) + int(count)
    return {"n_quant_linear": n, "modes": modes, "separate_calls": separate, "fused_calls": fused,
            "fallbacks": fallbacks,
            "note": "dispatch counts of real calls; fused_calls == 0 with fallbacks set means the separate "
                    "arm ran (several tokens always take it: the fused arm is the one-token decode GEMV)"}


def realized_bytes(module: Any) -> dict[str, int]:
    """Bytes a QuantLinear really stores: packed codes, scales, zero points, bias."""
    def nbytes(t: Any) -> int:
        return 0 if t is None else int(t.numel() * t.element_size())

    parts = {"packed_bytes": nbytes(module.packed), "scale_bytes": nbytes(module.scale),
             "zero_bytes": nbytes(module.zero), "bias_bytes": nbytes(module.bias)}
    parts["total_bytes"] = sum(parts.values())
    return parts


@dataclass
class QuantizeReport:
    """What ``quantize_model`` replaced, skipped and stores (``:492-511``)."""

    spec: dict[str, Any]
    replaced: dict[str, int] = field(default_factory=dict)
    skipped: list[str] = field(default_factory=list)
    realized_by_target: dict[str, dict[str, int]] = field(default_factory=dict)
    padding: dict[str, Any] = field(default_factory=dict)

    def to_dict(self) -> dict[str, Any]:
        return {
            "spec": self.spec,
            "replaced_per_target": self.replaced,
            "realized_bytes_total": sum(v["total_bytes"] for v in self.realized_by_target.values()),
            "realized_bytes_by_target": self.realized_by_target,
            "padding": self.padding,
            "skipped_linear_count": len(self.skipped),
            "skipped_linear_examples": self.skipped[:8],
        }


def _skip_reason(name: str, target: str | None, spec: SchemeSpec, layers: set | None, names: set | None) -> str | None:
    if target is None:
        return name
    if target not in spec.targets:
        return "%s (target=%s not in spec.targets)" % (name, target)
    if target == "lm_head" and spec.keep_lm_head_fp16:
        return "%s (keep_lm_head_fp16=True)" % name
    if names is not None and name not in names:
        return "%s (not in names=)" % name
    if layers is not None and _layer_index(name) not in layers:
        return "%s (layer=%s not in layers=%s)" % (name, _layer_index(name), sorted(layers))
    return None


def quantize_model(model: Any, spec: SchemeSpec, *, verbose: bool = False, layers: Any = None,
                   names: Any = None) -> tuple[Any, QuantizeReport]:
    """Replace ``model``'s ``nn.Linear`` modules by QuantLinear in place, chosen by
    their names (``classify_linear`` against ``spec.targets``, ``lm_head`` only
    without ``keep_lm_head_fp16``, optionally only ``layers`` / ``names``), as
    the reference's ``quantize_model`` (``:592-694``).  Every linear left alone
    is listed in the report with the reason.  Names are collected first and
    modules fetched one at a time, so each full-precision weight can be freed
    once its replacement exists.  The weights must be on a ROCm device (the
    quantiser runs there)."""
    report = QuantizeReport(spec=spec.to_dict())
    if not spec.enabled:
        return model, report
    layer_set = None if layers is None else {int(i) for i in layers}
    name_set = None if names is None else set(names)
    report.spec["layers"] = None if layer_set is None else sorted(layer_set)
    report.spec["names"] = None if name_set is None else sorted(name_set)
    todo = [n for n, m in model.named_modules() if n and isinstance(m, nn.Linear)]
    for name in todo:
        module = model.get_submodule(name)
        target = classify_linear(name)
        skip = _skip_reason(name, target, spec, layer_set, name_set)
        if skip is not None:
            report.skipped.append(skip)
            continue
        ql = QuantLinear.from_linear(module, spec, name=name)
        parent_name, _, leaf = name.rpartition(".")
        setattr(model.get_submodule(parent_name) if parent_name else model, leaf, ql)
        report.replaced[target] = report.replaced.get(target, 0) + 1
        bucket = report.realized_by_target.setdefault(target, {})
        for key, value in realized_bytes(ql).items():
            bucket[key] = bucket.get(key, 0) + value
        bucket["n_linear"] = bucket.get("n_linear", 0) + 1
        bucket["n_params"] = bucket.get("n_params", 0) + ql.out_features * ql.in_features
        bucket["n_params_padded"] = bucket.get("n_params_padded", 0) + ql.out_features * ql.padded_in
        if verbose:
            print("  quantized %s" % name)
    padded = sum(v["n_params_padded"] for v in report.realized_by_target.values())
    unpadded = sum(v["n_params"] for v in report.realized_by_target.values())
    report.padding = {
        "n_params_padded": padded,
        "n_params_unpadded": unpadded,
        "inflation_pct": round(100.0 * (padded - unpadded) / unpadded, 4) if unpadded else 0.0,
        "note": "padded columns are stored too; a byte count from unpadded parameters undercounts them",
    }
    return model, report
