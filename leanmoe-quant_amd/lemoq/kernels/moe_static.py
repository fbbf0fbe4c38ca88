"""MoE routing glue (``_route``) of the reference's ``moe_static``.

``_route(x, router_weight, *, top_k, norm_topk_prob)`` returns
``(logits, top_w, top_i)`` exactly as ``src/lemoq/kernels/moe_static.py:262-283``:
``logits = F.linear(x, W_r)`` in the activation dtype, fp32 softmax, top-k
(ties -> lowest index), optional renormalisation, ``top_w`` cast to ``x.dtype``.

For the decode shape (one fp16 token) the whole router is one HIP kernel
(``lemoq_router_topk_fused``: GEMV with fp32 accumulation and a single fp16
rounding of each logit, then softmax/top-k).  Several fp16 tokens run the
router linear as ``lemoq_gemm_f16`` (``lemoq.kernels.dequant_gemm.linear_f16``:
fp32 accumulation, one fp16 rounding, F.linear's contract in fp16) and then
the HIP top-k; other dtypes or widths (hidden % 64 != 0) use ATen's
``F.linear`` on the device, as the reference does, before the HIP top-k.
"""

from __future__ import annotations

from typing import Any

from lemoq import _hip

__all__ = ["FusedExperts", "_route", "fuse_experts"]


def fuse_experts(experts: Any):
    """Stack a list of per-expert MLPs (``gate_proj`` / ``up_proj`` / ``down_proj``
    linears, HF OLMoE 4.x's ``OlmoeSparseMoeBlock.experts``) into the packed
    layout: ``gate_up`` (E, 2F, H) with the gate rows first, ``down`` (E, H, F),
    as the reference's ``fuse_experts`` (``moe_static.py:106-122``).  Call once,
    outside capture; the stacked copies are new tensors on the experts' device."""
    import torch  # noqa: PLC0415

    from lemoq.kernels.moe_grouped_quant import FusedExperts  # noqa: PLC0415

    layers = list(experts)
    if not layers:
        raise ValueError("experts is empty")
    gate = torch.stack([e.gate_proj.weight.detach() for e in layers])
    up = torch.stack([e.up_proj.weight.detach() for e in layers])
    down = torch.stack([e.down_proj.weight.detach() for e in layers])
    return FusedExperts(gate_up=torch.cat([gate, up], dim=1).contiguous(), down=down.contiguous())


def __getattr__(name: str) -> Any:
    if name == "FusedExperts":  # the container lives with the quantised one
        from lemoq.kernels.moe_grouped_quant import FusedExperts  # noqa: PLC0415

        return FusedExperts
    raise AttributeError(name)


def _route(x: Any, router_weight: Any, *, top_k: int, norm_topk_prob: bool):
    import torch  # noqa: PLC0415
    import torch.nn.functional as F  # noqa: PLC0415

    if x.ndim != 2:
        raise ValueError("x must be (T, hidden), got %r" % (tuple(x.shape),))
    if router_weight.ndim != 2 or int(router_weight.shape[1]) != int(x.shape[1]):
        raise ValueError(
            "router_weight must be (E, hidden=%d), got %r"
            % (int(x.shape[1]), tuple(router_weight.shape))
        )
    _hip.require_rocm(x, router_weight, what="_route")
    t_tokens, hidden = int(x.shape[0]), int(x.shape[1])
    e = int(router_weight.shape[0])
    if type(top_k) is not int or not (0 < top_k <= e):
        raise ValueError("top_k=%r must be an integer in (0, %d]" % (top_k, e))
    fused_ok = (
        t_tokens == 1
        and x.dtype == torch.float16
        and router_weight.dtype == torch.float16
        and hidden % 16 == 0
        and hidden <= 8192
        and e <= 1024
        and top_k <= 64
    )
    if fused_ok:
        xc = x.contiguous()
        wc = router_weight.contiguous()
        if xc.data_ptr() % 16:
            xc = xc.clone()
        if wc.data_ptr() % 16:
            wc = wc.clone()
        logits = torch.empty((1, e), dtype=torch.float16, device=x.device)
        top_w = torch.empty((1, top_k), dtype=torch.float16, device=x.device)
        top_i = torch.empty((1, top_k), dtype=torch.int64, device=x.device)
        _hip.call(
            "lemoq_router_topk_fused",
            _hip.ptr(xc),
            None,
            0.0,
            hidden,
            _hip.ptr(wc),
            e,
            top_k,
            1 if norm_topk_prob else 0,
            None,
            _hip.ptr(logits),
            None,
            _hip.ptr(top_w),
            _hip.ptr(top_i),
            _hip.stream_of(x.device),
        )
        return logits, top_w, top_i
    from lemoq.kernels.routing import routing_softmax_topk  # noqa: PLC0415

    if x.dtype == torch.float16 and router_weight.dtype == torch.float16 and hidden % 64 == 0:
        from lemoq.kernels.dequant_gemm import linear_f16  # noqa: PLC0415

        xc, wc = x.contiguous(), router_weight.contiguous()
        if xc.data_ptr() % 16:
            xc = xc.clone()
        if wc.data_ptr() % 16:
            wc = wc.clone()
        logits = linear_f16(xc, wc)
    else:
        logits = F.linear(x, router_weight)
    top_w, top_i = routing_softmax_topk(logits, top_k=top_k, norm_topk_prob=norm_topk_prob)
    return logits, top_w.to(x.dtype), top_i
