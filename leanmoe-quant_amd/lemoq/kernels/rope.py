"""Rotary position embedding for the decode shape (``lemoq_rope``), and the cos/sin table.

``apply_rotary_pos_emb_fused(q, k, cos, sin, position_ids=None, unsqueeze_dim=1)``
replaces the reference's fused RoPE (``src/lemoq/kernels/rope.py:154-203``):
``out = x*cos + rotate_half(x)*sin`` with ``rotate_half(x) = cat(-x2, x1)``,
computed in fp32 and rounded to fp16, on ``(1, H, 1, D)`` q and k (strided
views allowed).  Shapes other than the decode shape raise (the reference hands
them to HF; this build has no host path).

``rotary_cos_sin(positions, head_dim, theta)`` builds the fp16 cos/sin rows of
HF ``OlmoeRotaryEmbedding`` (``inv_freq = 1/theta^(arange(0, D, 2)/D)`` in fp32,
``freqs = inv_freq * pos``, ``emb = cat(freqs, freqs)``, ``cos/sin`` in fp32
cast to fp16).  It is a one-time table build at model set-up, evaluated with
torch on the host so every run uses the same table; the decode step reads the
row of the current position on the device.
"""

from __future__ import annotations

from typing import Any

from lemoq import _hip

__all__ = ["apply_rotary_pos_emb_fused", "fused_rope_available", "rotary_cos_sin"]


def fused_rope_available() -> bool:
    return _hip.library_available()


def rotary_cos_sin(positions: Any, head_dim: int, theta: float = 10000.0):
    """``positions`` (P,) int -> ``(cos, sin)`` each (P, head_dim) fp16 (CPU tensors)."""
    import torch  # noqa: PLC0415

    pos = torch.as_tensor(positions, dtype=torch.int64).reshape(-1).cpu()
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = inv_freq[None, :, None].float() @ pos[None, None, :].float()  # (1, D/2, P)
    freqs = freqs.transpose(1, 2)[0]  # (P, D/2)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(torch.float16), emb.sin().to(torch.float16)


def _decode_shape_ok(q: Any, k: Any, cos_u: Any, sin_u: Any) -> bool:
    import torch  # noqa: PLC0415

    if q.ndim != 4 or k.ndim != 4:
        return False
    if q.dtype != torch.float16 or any(t.dtype != q.dtype for t in (k, cos_u, sin_u)):
        return False
    if q.shape[0] != 1 or k.shape[0] != 1 or q.shape[2] != 1 or k.shape[2] != 1:
        return False
    d = int(q.shape[3])
    if int(k.shape[3]) != d or d % 2 != 0 or d < 2 or d > 1024:
        return False
    if tuple(cos_u.shape) != (1, 1, 1, d) or tuple(sin_u.shape) != (1, 1, 1, d):
        return False
    return cos_u.stride(-1) == sin_u.stride(-1)


def apply_rotary_pos_emb_fused(
    q: Any, k: Any, cos: Any, sin: Any, position_ids: Any = None, unsqueeze_dim: int = 1
) -> tuple[Any, Any]:
    import torch  # noqa: PLC0415

    if position_ids is not None:
        raise NotImplementedError("position_ids must be None (cos/sin already carry the position)")
    cos_u = cos.unsqueeze(unsqueeze_dim)
    sin_u = sin.unsqueeze(unsqueeze_dim)
    if not _decode_shape_ok(q, k, cos_u, sin_u):
        raise NotImplementedError(
            "fused RoPE handles the fp16 decode shape (1,H,1,D) with (1,1,D) cos/sin only"
        )
    _hip.require_rocm(q, k, cos_u, sin_u, what="apply_rotary_pos_emb_fused")
    d = int(q.shape[3])
    qo = torch.empty_like(q)
    ko = torch.empty_like(k)
    st = _hip.stream_of(q.device)
    for x, out in ((q, qo), (k, ko)):
        _hip.call(
            "lemoq_rope",
            _hip.ptr(x), int(x.stride(1)), int(x.stride(3)), int(x.shape[1]), d,
            _hip.ptr(cos_u), _hip.ptr(sin_u), int(cos_u.stride(3)),
            _hip.ptr(out), int(out.stride(1)), int(out.stride(3)), st,
        )
    return qo, ko


def warm(*, heads: int = 16, kv_heads: int = 4, head_dim: int = 128, device: Any = None) -> None:
    """One real launch before graph capture, with the reference's signature and
    defaults (src/lemoq/kernels/rope.py:206): rotates (1, heads, 1, head_dim) q
    and (1, kv_heads, 1, head_dim) k by the angles of position 1 at base 10000
    (the (1, 1, head_dim) cos/sin of a real decode step), then synchronises."""
    import torch  # noqa: PLC0415

    dev = torch.device(device if device is not None else "cuda")
    half = head_dim // 2
    inv_freq = 10000.0 ** (-torch.arange(half, dtype=torch.float32) / half)
    ang = torch.cat((inv_freq, inv_freq)).view(1, 1, head_dim)
    cos, sin = (f(ang).to(dev, torch.float16) for f in (torch.cos, torch.sin))
    q = torch.ones((1, heads, 1, head_dim), dtype=torch.float16, device=dev)
    k = torch.ones((1, kv_heads, 1, head_dim), dtype=torch.float16, device=dev)
    apply_rotary_pos_emb_fused(q, k, cos, sin)
    torch.cuda.synchronize(dev)
