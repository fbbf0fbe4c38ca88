"""Grouped MoE decode on w8 (and 4-bit) weights: gate/up + SiLU and down + weighted sum.

Operator surface of the reference's ``src/lemoq/kernels/moe_grouped_quant.py``:

* ``QuantFusedExperts`` (``:72-188``) — packed codes + per-group fp16 scales,
  ``packed_gate_up`` (E, 2F, H) int8 with gate rows [0, F) and up rows [F, 2F),
  ``packed_down`` (E, H, F) int8, ``scale_gate_up`` (E, 2F, H/g),
  ``scale_down`` (E, H, F/g), groups along the last (K) dimension; at
  ``bits=4`` the codes are int4 packed two per byte (uint8, last dim halved).
* ``quantize_fused_experts`` (``:191-244``) — RTN w8 or w4 of the fused fp
  weights (on the device, ``lemoq_rtn_quantize``).
* ``grouped_moe_forward_quant`` (``:411-559``) — ``(H,)`` token + ``(K,)`` expert
  ids + ``(K,)`` routing weights -> ``(H,)``; two HIP launches
  (``lemoq_moe_gate_up_w8``, ``lemoq_moe_down_w8``; ``_w4`` at 4 bits), the reference's SPLIT_K
  reduction kernel is folded into the down kernel's fixed-order epilogue.
* ``static_moe_forward_grouped_quant`` (``:562-601``) — the MoE block glue with
  ``_route``.

Numerics as the reference kernels (``_grouped_triton.py:249-398``): fp32
accumulation, ``act`` rounded to fp16 between the two GEMVs, the routing
weight taken as fp16 and applied in fp32, fp16 output.  ``backend`` accepts
``"auto"``, ``"hip"`` and ``"triton"`` (alias, for call-site compatibility);
``"oracle"`` raises — the CPU restatement is test infrastructure, not a
product path.
"""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass
from typing import Any

from lemoq import _hip

__all__ = [
    "FusedExperts",
    "QuantFusedExperts",
    "dequantize_fused_experts",
    "grouped_moe_forward_quant",
    "quant_launch_plan",
    "quantize_fused_experts",
    "quantized_grouped_available",
    "static_moe_forward_grouped_quant",
]

PARITY_GATE = {"tol_atol": 1e-3, "tol_rtol": 1e-3, "tol_slack": 1.5}
_MAX_OFFSET = 2**40  # 64-bit offsets in the kernels; guard absurd sizes only

# Launch geometry of the HIP kernels (fixed; see csrc/moe.hip).
GATE_UP_ROWS_PER_WAVE = 2
DOWN_ROWS_PER_BLOCK = 4


@dataclass
class FusedExperts:
    """fp weights of all experts stacked: gate_up (E, 2F, H), down (E, H, F)."""

    gate_up: Any
    down: Any


@dataclass
class QuantFusedExperts:
    packed_gate_up: Any
    scale_gate_up: Any
    packed_down: Any
    scale_down: Any
    bits: int
    group_size: int

    @property
    def num_experts(self) -> int:
        return int(self.packed_gate_up.shape[0])

    @property
    def ffn(self) -> int:
        return int(self.packed_gate_up.shape[1]) // 2

    @property
    def hidden(self) -> int:
        return int(self.packed_gate_up.shape[-1]) * (8 // int(self.bits))

    # The four device tensors, in the order they are laid out in HBM.
    _TENSORS = ("packed_gate_up", "scale_gate_up", "packed_down", "scale_down")

    def nbytes(self) -> int:
        """Bytes of codes and scales together (what one full pass over every
        expert reads)."""
        return sum(getattr(self, f).numel() * getattr(self, f).element_size() for f in self._TENSORS)

    def _dequant_rows(self, codes: Any, scale: Any, rows: int, width: int, dtype: Any) -> Any:
        """(rows, width) weights of stacked packed rows, ``code * scale`` in fp32
        (``lemoq_dequant_q``), rounded once to ``dtype`` when given
        (``src/lemoq/kernels/moe_grouped_quant.py:145-157``)."""
        import torch  # noqa: PLC0415

        from lemoq.quant.formats import QFMT_W4, QFMT_W8, dequantize  # noqa: PLC0415

        out = dtype if dtype in (torch.float16, torch.float32) else torch.float32
        w = dequantize(codes.reshape(rows, -1), scale.reshape(rows, -1), None,
                       fmt=QFMT_W8 if int(self.bits) == 8 else QFMT_W4, group_size=int(self.group_size),
                       k_out=width, dtype=out)
        return w if dtype is None or dtype == out else w.to(dtype)

    def dequant_gate_up(self, dtype: Any = None) -> Any:
        e, rows = int(self.packed_gate_up.shape[0]), int(self.packed_gate_up.shape[1])
        return self._dequant_rows(self.packed_gate_up, self.scale_gate_up, e * rows, self.hidden,
                                  dtype).reshape(e, rows, self.hidden)

    def dequant_down(self, dtype: Any = None) -> Any:
        e, rows = int(self.packed_down.shape[0]), int(self.packed_down.shape[1])
        return self._dequant_rows(self.packed_down, self.scale_down, e * rows, self.ffn, dtype).reshape(
            e, rows, self.ffn)

    def dequant_gate_up_expert(self, index: int, dtype: Any = None) -> Any:
        """One expert's (2F, H) gate/up weight (without dequantising the others)."""
        return self._dequant_rows(self.packed_gate_up[index], self.scale_gate_up[index], 2 * self.ffn, self.hidden,
                                  dtype)

    def dequant_down_expert(self, index: int, dtype: Any = None) -> Any:
        return self._dequant_rows(self.packed_down[index], self.scale_down[index], self.hidden, self.ffn, dtype)

    def to(self, device: Any = None, dtype: Any = None) -> "QuantFusedExperts":
        """Copy to ``device`` (contiguous).  Codes keep their storage type and scales fp16, so a
        dtype is refused, also when passed positionally as ``to(torch.float32)``:
        converting would undo the quantisation."""
        import torch  # noqa: PLC0415

        if dtype is None and isinstance(device, torch.dtype):
            device, dtype = None, device
        if dtype is not None:
            raise ValueError("QuantFusedExperts keeps int8 codes and fp16 scales; dtype=%r refused "
                             "(quantize again for another precision)" % (dtype,))
        if device is None:
            return self
        moved = {f: getattr(self, f).to(device=device).contiguous() for f in self._TENSORS}
        return dataclasses.replace(self, **moved)


def quantize_fused_experts(fused: Any, *, bits: int = 8, group_size: int = 128) -> QuantFusedExperts:
    """RTN-quantize ``fused.gate_up`` (E, 2F, H) and ``fused.down`` (E, H, F) on the
    device, symmetric, 8-bit (int8 codes) or 4-bit (int4 codes packed two per byte)."""
    from lemoq.quant import rtn  # noqa: PLC0415

    if bits not in (4, 8):
        raise NotImplementedError("grouped quantization implements 4/8-bit, got %r" % (bits,))
    if group_size <= 0:
        raise ValueError("group_size must be > 0")
    if bits == 4 and group_size % 2 != 0:
        raise ValueError("4-bit packing needs an even group_size, got %d" % group_size)
    gate_up, down = fused.gate_up, fused.down
    hidden = int(gate_up.shape[2])
    ffn = int(down.shape[2])
    for name, dim in (("hidden", hidden), ("ffn", ffn)):
        if dim % group_size != 0:
            raise NotImplementedError(
                "%s=%d is not divisible by group_size=%d (the grouped path does not pad)"
                % (name, dim, group_size)
            )
    q_gu = rtn.quantize_rtn(gate_up.reshape(-1, hidden), bits=bits, group_size=group_size)
    q_d = rtn.quantize_rtn(down.reshape(-1, ffn), bits=bits, group_size=group_size)
    e, rows_gu = int(gate_up.shape[0]), int(gate_up.shape[1])
    rows_d = int(down.shape[1])
    per = 1 if bits == 8 else 2  # codes per stored byte
    return QuantFusedExperts(
        packed_gate_up=q_gu["packed"].reshape(e, rows_gu, hidden // per).contiguous(),
        scale_gate_up=q_gu["scale_f16"].reshape(e, rows_gu, hidden // group_size).contiguous(),
        packed_down=q_d["packed"].reshape(e, rows_d, ffn // per).contiguous(),
        scale_down=q_d["scale_f16"].reshape(e, rows_d, ffn // group_size).contiguous(),
        bits=int(bits),
        group_size=int(group_size),
    )


def quantized_grouped_available() -> bool:
    """True when the HIP library is built and a ROCm device is visible (never raises)."""
    try:
        import torch  # noqa: PLC0415

        return _hip.library_available() and bool(torch.cuda.is_available())
    except Exception:  # noqa: BLE001
        return False


def dequantize_fused_experts(q: "QuantFusedExperts", dtype: Any = None) -> FusedExperts:
    """``QuantFusedExperts`` -> ``FusedExperts`` with the dense weights (fp32, or
    ``dtype``), dequantised on the device (``QuantFusedExperts.dequant_gate_up`` /
    ``dequant_down``), as the reference's ``dequantize_fused_experts``
    (``moe_grouped_quant.py:247-254``)."""
    return FusedExperts(gate_up=q.dequant_gate_up(dtype=dtype), down=q.dequant_down(dtype=dtype))


def _cdiv(a: int, b: int) -> int:
    return -(-int(a) // int(b))


def quant_launch_plan(
    q: QuantFusedExperts,
    *,
    top_k: int,
    config: dict[str, Any] | None = None,
    for_kernel: bool = True,
) -> dict[str, Any]:
    """Grids and buffer shapes of the two HIP launches, and the format checks.

    Pure host arithmetic (testable without a GPU), as the reference's
    ``quant_launch_plan`` (``moe_grouped_quant.py:289-379``).  Checks, always:
    bits 4 or 8 with codes stored as int8 / packed uint8, contiguous tensors,
    hidden/ffn divisible by group_size; with ``for_kernel``: group_size a
    multiple of a lane's slice (16 codes at 8 bits, 32 at 4) and hidden, ffn
    <= 8192 (a slice never straddles a group; one row fits the register tiling).
    """
    import torch  # noqa: PLC0415

    del config
    bits = int(q.bits)
    if bits not in (4, 8):
        raise NotImplementedError("grouped path implements 4/8-bit, got %d" % bits)
    if top_k <= 0:
        raise ValueError("top_k must be > 0")
    e = int(q.packed_gate_up.shape[0])
    ffn = int(q.packed_gate_up.shape[1]) // 2
    hidden = q.hidden
    for name, tensor in (
        ("packed_gate_up", q.packed_gate_up),
        ("scale_gate_up", q.scale_gate_up),
        ("packed_down", q.packed_down),
        ("scale_down", q.scale_down),
    ):
        if not tensor.is_contiguous():
            raise ValueError("%s must be contiguous" % name)
        if int(tensor.numel()) >= _MAX_OFFSET:
            raise ValueError("%s is too large" % name)
    per = 8 // bits  # codes per stored byte
    want = torch.int8 if bits == 8 else torch.uint8
    if q.packed_gate_up.dtype != want or q.packed_down.dtype != want:
        raise ValueError("%d-bit codes must be %s" % (bits, want))
    if tuple(q.packed_down.shape) != (e, hidden, ffn // per):
        raise ValueError(
            "packed_down must be (E=%d, H=%d, F/%d=%d), got %r"
            % (e, hidden, per, ffn // per, tuple(q.packed_down.shape))
        )
    group = int(q.group_size)
    for name, dim in (("hidden", hidden), ("ffn", ffn)):
        if dim % group != 0:
            raise ValueError("%s=%d not divisible by group_size=%d" % (name, dim, group))
    if tuple(q.scale_gate_up.shape) != (e, 2 * ffn, hidden // group):
        raise ValueError("scale_gate_up has shape %r" % (tuple(q.scale_gate_up.shape),))
    if tuple(q.scale_down.shape) != (e, hidden, ffn // group):
        raise ValueError("scale_down has shape %r" % (tuple(q.scale_down.shape),))
    plan: dict[str, Any] = {
        "hidden": hidden,
        "ffn": ffn,
        "top_k": int(top_k),
        "num_experts": e,
        "gate_up_act": {
            "grid": (_cdiv(ffn, 4 * GATE_UP_ROWS_PER_WAVE), int(top_k)),
            "block": 256,
            "act_shape": (int(top_k), ffn),
        },
        "down_sum": {
            "grid": (_cdiv(hidden, DOWN_ROWS_PER_BLOCK),),
            "block": 512,
            "out_shape": (hidden,),
        },
        "kernel_count": 2,
        "quant": {"bits": bits, "group_size": group, "for_kernel": bool(for_kernel)},
        "kernels": ("lemoq_moe_gate_up_w8", "lemoq_moe_down_w8") if bits == 8 else
                   ("lemoq_moe_gate_up_w4", "lemoq_moe_down_w4"),
    }
    if for_kernel:
        step = 16 if bits == 8 else 32  # codes per 16-byte lane slice
        if group % step != 0:
            raise ValueError("group_size=%d must be a multiple of %d for the %d-bit HIP kernels"
                             % (group, step, bits))
        if hidden > 8192 or ffn > 8192 or hidden % step or ffn % step:
            raise NotImplementedError("hidden and ffn must be multiples of %d and <= 8192" % step)
        if int(top_k) > 64:
            raise NotImplementedError("top_k <= 64 is supported")
    return plan


def _check_backend(backend: str) -> None:
    if backend not in ("auto", "hip", "triton", "oracle"):
        raise ValueError("unknown backend %r" % (backend,))
    if backend == "oracle":
        raise NotImplementedError(
            "backend='oracle' is the CPU restatement kept with the tests (oracle/); "
            "the MI355X build has no CPU compute path"
        )


def grouped_moe_forward_quant(
    x: Any,
    q: QuantFusedExperts,
    ids: Any,
    top_w: Any,
    *,
    config: dict[str, Any] | None = None,
    backend: str = "auto",
    residual: Any = None,
) -> Any:
    """``(H,)`` hidden state, ``(K,)`` expert ids, ``(K,)`` routing weights -> ``(H,)`` fp16.

    ``residual`` (this build's extension, default None): when given, returns
    ``fp16(fp16(moe) + residual)`` — the decoder layer's residual add folded
    into the down kernel with the intermediate fp16 rounding kept.
    """
    import torch  # noqa: PLC0415

    _check_backend(backend)
    if q.scale_gate_up.dtype != torch.float16:
        raise NotImplementedError(
            "grouped kernels store fp16 and take fp16 scales; got %s"
            % str(q.scale_gate_up.dtype).replace("torch.", "")
        )
    xf = x.reshape(-1)
    if xf.dtype != q.scale_gate_up.dtype:
        xf = xf.to(q.scale_gate_up.dtype)
    xf = xf.contiguous()
    idx = ids.reshape(-1)
    if idx.dtype != torch.int64:
        idx = idx.to(torch.int64)
    idx = idx.contiguous()
    wsum = top_w.reshape(-1)
    if wsum.dtype != xf.dtype:
        wsum = wsum.to(xf.dtype)
    wsum = wsum.contiguous()
    top_k = int(idx.numel())
    plan = quant_launch_plan(q, top_k=top_k, config=config, for_kernel=True)
    hidden, ffn = int(plan["hidden"]), int(plan["ffn"])
    if int(xf.numel()) != hidden:
        raise ValueError(
            "grouped_moe_forward_quant handles one token: x has %d elements, hidden is %d"
            % (int(xf.numel()), hidden)
        )
    if int(wsum.numel()) != top_k:
        raise ValueError("top_w has %d entries for %d slots" % (int(wsum.numel()), top_k))
    if residual is not None:
        residual = residual.reshape(-1)
        if int(residual.numel()) != hidden or residual.dtype != torch.float16:
            raise ValueError("residual must be (H,) fp16")
        residual = residual.contiguous()
    _hip.require_rocm(
        xf, idx, wsum, q.packed_gate_up, q.scale_gate_up, q.packed_down, q.scale_down, residual,
        what="grouped_moe_forward_quant",
    )
    dev = xf.device
    st = _hip.stream_of(dev)
    act = torch.empty(plan["gate_up_act"]["act_shape"], dtype=torch.float16, device=dev)
    out = torch.empty((hidden,), dtype=torch.float16, device=dev)
    _hip.call(
        plan["kernels"][0],
        _hip.ptr(xf),
        _hip.ptr(q.packed_gate_up),
        _hip.ptr(q.scale_gate_up),
        _hip.ptr(idx),
        top_k,
        q.num_experts,
        ffn,
        hidden,
        int(q.group_size),
        _hip.ptr(act),
        st,
    )
    _hip.call(
        plan["kernels"][1],
        _hip.ptr(act),
        _hip.ptr(q.packed_down),
        _hip.ptr(q.scale_down),
        _hip.ptr(idx),
        _hip.ptr(wsum),
        top_k,
        q.num_experts,
        hidden,
        ffn,
        int(q.group_size),
        _hip.ptr(residual),
        _hip.ptr(out),
        st,
    )
    return out


def grouped_gate_up_act_quant(x: Any, q: QuantFusedExperts, ids: Any) -> Any:
    """The first launch alone: ``act (K, F) fp16`` (exposed for per-kernel tests)."""
    import torch  # noqa: PLC0415

    xf = x.reshape(-1).to(torch.float16).contiguous()
    idx = ids.reshape(-1).to(torch.int64).contiguous()
    plan = quant_launch_plan(q, top_k=int(idx.numel()), for_kernel=True)
    if int(xf.numel()) != plan["hidden"]:
        raise ValueError("x has %d elements, hidden is %d" % (int(xf.numel()), plan["hidden"]))
    _hip.require_rocm(xf, idx, q.packed_gate_up, q.scale_gate_up, what="grouped_gate_up_act_quant")
    act = torch.empty(plan["gate_up_act"]["act_shape"], dtype=torch.float16, device=xf.device)
    _hip.call(
        plan["kernels"][0],
        _hip.ptr(xf),
        _hip.ptr(q.packed_gate_up),
        _hip.ptr(q.scale_gate_up),
        _hip.ptr(idx),
        int(idx.numel()),
        q.num_experts,
        plan["ffn"],
        plan["hidden"],
        int(q.group_size),
        _hip.ptr(act),
        _hip.stream_of(xf.device),
    )
    return act


def static_moe_forward_grouped_quant(
    hidden_states: Any,
    router_weight: Any,
    q: QuantFusedExperts,
    *,
    top_k: int,
    norm_topk_prob: bool,
    act_fn: Any,
    config: dict[str, Any] | None = None,
    backend: str = "auto",
) -> tuple[Any, Any]:
    """``OlmoeSparseMoeBlock.forward`` for one token: returns ``(out, router_logits)``."""
    from lemoq.kernels.moe_static import _route  # noqa: PLC0415

    _check_act_fn(act_fn)
    _check_backend(backend)
    shape = tuple(hidden_states.shape)
    hidden = shape[-1]
    tokens = 1
    for s in shape[:-1]:
        tokens *= s
    if tokens != 1:
        raise NotImplementedError("the grouped decode path handles one token (got %d)" % tokens)
    x = hidden_states.reshape(tokens, hidden)
    logits, top_w, top_i = _route(x, router_weight, top_k=top_k, norm_topk_prob=norm_topk_prob)
    out = grouped_moe_forward_quant(
        x, q, top_i.reshape(-1), top_w.reshape(-1), config=config, backend=backend
    )
    return out.reshape(*shape), logits


def _check_act_fn(act_fn: Any) -> None:
    """The kernels fuse SiLU; any other activation is refused, not silently replaced."""
    if act_fn is None:
        return
    name = getattr(act_fn, "__name__", "") or type(act_fn).__name__
    if name.lower() in ("silu", "siluactivation"):
        return
    raise NotImplementedError("the grouped kernels fuse silu; act_fn=%r is not silu" % (act_fn,))
