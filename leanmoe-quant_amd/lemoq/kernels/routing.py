"""Router softmax + top-k on the device (``lemoq_route_topk``).

Replaces ``routing_softmax_topk`` (``src/lemoq/kernels/_routing_triton.py:88-130``):
``(T, E)`` logits -> fp32 softmax -> top-``k`` by probability with ties going
to the lowest expert index -> optional renormalisation over the selected
``k``.  Returns ``(top_w fp32 (T, k), top_i int64 (T, k))``.  Empty input
returns empty outputs without touching the device; a CPU tensor raises.
"""

from __future__ import annotations

from typing import Any

from lemoq import _hip

__all__ = ["routing_softmax_topk", "MAX_EXPERTS"]

MAX_EXPERTS = 1024


def routing_softmax_topk(logits: Any, *, top_k: int, norm_topk_prob: bool = False) -> tuple[Any, Any]:
    import torch  # noqa: PLC0415

    if not torch.is_tensor(logits):
        raise TypeError("logits must be a tensor")
    if logits.ndim != 2:
        raise ValueError("logits must be (T, E), got shape %s" % (tuple(logits.shape),))
    t_tokens, e = int(logits.shape[0]), int(logits.shape[1])
    if type(top_k) is not int or not (0 < top_k <= e):
        raise ValueError("top_k=%r must be an integer in (0, %d]" % (top_k, e))
    if not logits.is_floating_point():
        raise ValueError("logits must be a floating-point tensor")
    if e > MAX_EXPERTS or top_k > 64:
        raise NotImplementedError("E <= %d and top_k <= 64 are supported" % MAX_EXPERTS)
    if logits.dtype not in (torch.float16, torch.float32):
        raise NotImplementedError("logits must be fp16 or fp32, got %s" % logits.dtype)
    top_w = torch.empty((t_tokens, top_k), dtype=torch.float32, device=logits.device)
    top_i = torch.empty((t_tokens, top_k), dtype=torch.int64, device=logits.device)
    if t_tokens == 0:
        return top_w, top_i
    if not logits.is_cuda:
        raise RuntimeError("routing_softmax_topk requires a ROCm device tensor (no CPU path)")
    contiguous = logits if logits.is_contiguous() else logits.contiguous()
    _hip.call(
        "lemoq_route_topk",
        _hip.ptr(contiguous),
        1 if contiguous.dtype == torch.float16 else 0,
        t_tokens,
        e,
        int(contiguous.stride(0)),
        top_k,
        1 if norm_topk_prob else 0,
        _hip.ptr(top_w),
        _hip.ptr(top_i),
        _hip.stream_of(logits.device),
    )
    return top_w, top_i
