"""GPU parity of the one-launch attention half of a decoder layer
(lemoq_attn_layer_i8) against the three launches it replaces:
lemoq_attn_split_fused_i8 -> lemoq_attn_merge_o_proj_w8 ->
lemoq_router_logits_resid (themselves pinned to the oracle in
test_gpu_attn_fused.py, test_gpu_ops.py and test_gpu_decode.py).

The fused launch's workgroups hand the split partials and the o_proj partial
sums to each other inside the launch (coherent stores, counters, bounded
waits), with the arithmetic of the three launches, so every output must be
equal BIT FOR BIT: router logits, the residual h', the normed xn, the o_proj
partials, the split partials and the KV-INT8 bytes written for the new token.
The sync workspace must be zero again after every successful launch.

Failure handling is forced from the host: with a time limit of 0 the waits
give up, the status word carries LEMOQ_SYNC_TIMEOUT_BIT and the launch still
completes; after lemoq_sync_reset the next launch is exact again.
"""

from __future__ import annotations

import math

import pytest
import torch

from helpers import randn
from oracle import ops
from oracle import quant as oq

pytestmark = pytest.mark.gpu

LOG2E = 1.4426950408889634
SYNC_WORDS = 16384  # LEMOQ_SYNC_WORDS


def _inputs(heads, D, S, H, E, seed):
    HD = heads * D
    g = torch.Generator().manual_seed(seed)
    x = {
        "qkv": (torch.randn((3 * HD,), generator=g) * 2).to(torch.float16),
        "qn": (torch.rand((HD,), generator=g) + 0.5).to(torch.float16),
        "kn": (torch.rand((HD,), generator=g) + 0.5).to(torch.float16),
        "h": torch.randn((H,), generator=g).to(torch.float16),
        "ln": (torch.rand((H,), generator=g) + 0.5).to(torch.float16),
        "router": (torch.randn((E, H), generator=g) * 0.02).to(torch.float16),
    }
    k = torch.randn((heads, S, D), generator=g).to(torch.float16)
    v = torch.randn((heads, S, D), generator=g).to(torch.float16)
    kc, ks = oq.kv_quantize_rows(k.numpy())
    vc, vs = oq.kv_quantize_rows(v.numpy())
    x["cache"] = {n: torch.from_numpy(a) for n, a in (("kc", kc), ("ks", ks), ("vc", vc), ("vs", vs))}
    q = oq.rtn_quantize_w8(randn(H, HD, seed=seed + 1, std=0.02).numpy(), 128)
    x["o_codes"] = torch.from_numpy(q["codes_padded"])
    x["o_scale"] = torch.from_numpy(q["scale_f16"])
    cos, sin = ops.rotary_cos_sin(torch.arange(S), D, 1e4)
    x["cos"], x["sin"] = cos.contiguous(), sin.contiguous()
    return x


def _bufs(dev, heads, D, ns, H, E, cache):
    HD = heads * D
    nan = float("nan")
    return {
        "c": {n: t.clone().to(dev) for n, t in cache.items()},
        "m": torch.full((heads * ns,), nan, dtype=torch.float32, device=dev),
        "l": torch.full((heads * ns,), nan, dtype=torch.float32, device=dev),
        "acc": torch.full((heads * ns * D,), nan, dtype=torch.float32, device=dev),
        "part": torch.full((HD // 512, H), nan, dtype=torch.float32, device=dev),
        "h_out": torch.full((H,), nan, dtype=torch.float16, device=dev),
        "xn": torch.full((H,), nan, dtype=torch.float16, device=dev),
        "logits": torch.full((E,), nan, dtype=torch.float16, device=dev),
    }


def _run(hip, dev, x, pos, heads, D, S, ns, H, E, *, fused, sync=None, timeout_us=200_000):
    P, st = hip.ptr, hip.stream_of(dev)
    d = {n: x[n].to(dev) for n in ("qkv", "qn", "kn", "h", "ln", "router", "o_codes", "o_scale", "cos", "sin")}
    b = _bufs(dev, heads, D, ns, H, E, x["cache"])
    c = b["c"]
    posd = torch.tensor([pos], dtype=torch.int64, device=dev)
    qk_scale = (1.0 / math.sqrt(D)) * LOG2E
    if fused:
        hip.call("lemoq_attn_layer_i8", P(d["qkv"]), heads, D, P(d["qn"]), P(d["kn"]), 1e-5, P(d["cos"]),
                 P(d["sin"]), P(posd), P(c["kc"]), P(c["ks"]), P(c["vc"]), P(c["vs"]), S * D, S, ns, qk_scale,
                 P(b["m"]), P(b["l"]), P(b["acc"]), P(d["o_codes"]), P(d["o_scale"]), H, 128, P(b["part"]),
                 P(d["h"]), P(d["ln"]), P(d["router"]), E, P(b["h_out"]), P(b["xn"]), P(b["logits"]), P(sync),
                 timeout_us, st)
    else:
        hip.call("lemoq_attn_split_fused_i8", P(d["qkv"]), heads, D, P(d["qn"]), P(d["kn"]), 1e-5, P(d["cos"]),
                 P(d["sin"]), P(posd), P(c["kc"]), P(c["ks"]), P(c["vc"]), P(c["vs"]), S * D, S, ns, qk_scale,
                 P(b["m"]), P(b["l"]), P(b["acc"]), st)
        hip.call("lemoq_attn_merge_o_proj_w8", P(b["m"]), P(b["l"]), P(b["acc"]), heads, ns, D, P(d["o_codes"]),
                 P(d["o_scale"]), H, 128, P(b["part"]), st)
        hip.call("lemoq_router_logits_resid", P(b["part"]), heads * D // 512, P(d["h"]), P(d["ln"]), 1e-5, H,
                 P(d["router"]), E, P(b["h_out"]), P(b["xn"]), P(b["logits"]), st)
    torch.cuda.synchronize()
    out = {n: t.cpu() for n, t in b.items() if n != "c"}
    out.update({n: t.cpu() for n, t in c.items()})
    return out


def _bitwise(a, b, what):
    for n in a:
        x, y = a[n], b[n]
        if x.dtype == torch.float16:
            x, y = x.view(torch.int16), y.view(torch.int16)
        elif x.dtype == torch.float32:
            x, y = x.view(torch.int32), y.view(torch.int32)
        assert torch.equal(x, y), "%s: %s differs" % (what, n)


CASES = [
    # heads, D, S, pos, ns, H, E
    (16, 128, 1100, 1060, 16, 2048, 64),   # the OLMoE step at ctx ~1k: 256 workgroups = 256 o_proj tiles
    (16, 128, 4200, 4132, 16, 2048, 64),   # ctx ~4k
    (16, 128, 1100, 0, 16, 2048, 64),      # first token: 15 empty splits
    (16, 128, 300, 77, 4, 2048, 64),       # 64 workgroups: 4 o_proj tiles each
    (8, 128, 1200, 1190, 32, 2048, 64),    # 8 heads (2 partial rows), 32 splits (64-split merge)
    (16, 128, 600, 333, 8, 4096, 128),     # hidden 4096, 128 experts
    (4, 128, 500, 499, 16, 2048, 8),       # 1 head group, 8 experts (2 router workgroups)
]


@pytest.mark.parametrize("heads,D,S,pos,ns,H,E", CASES)
def test_attn_layer_equals_three_launches_bitwise(heads, D, S, pos, ns, H, E, dev):
    from lemoq import _hip

    print("case: attn_layer heads=%d S=%d pos=%d ns=%d H=%d E=%d" % (heads, S, pos, ns, H, E), flush=True)
    assert int(_hip.load().lemoq_attn_layer_check(heads, D, ns, H, 128, E)) == 0
    x = _inputs(heads, D, S, H, E, seed=heads + S + pos)
    sync = torch.zeros((SYNC_WORDS,), dtype=torch.int32, device=dev)
    ref = _run(_hip, dev, x, pos, heads, D, S, ns, H, E, fused=False)
    for rep in range(2):  # the workspace returns to zero, so a second launch is exact too
        got = _run(_hip, dev, x, pos, heads, D, S, ns, H, E, fused=True, sync=sync)
        assert int(sync[0].item()) == 0, "status %d" % int(sync[0].item())
        assert int(torch.count_nonzero(sync)) == 0, "sync workspace not returned to zero"
        _bitwise(ref, got, "rep %d" % rep)


def test_attn_layer_forced_timeout_completes_and_reports(dev):
    """A time limit of 0: the waits give up at once, the launch still completes,
    the status carries the timeout bit; reset, then a normal launch is exact."""
    from lemoq import _hip

    heads, D, S, pos, ns, H, E = 16, 128, 1100, 1060, 16, 2048, 64
    print("case: attn_layer forced timeout", flush=True)
    x = _inputs(heads, D, S, H, E, seed=5)
    sync = torch.zeros((SYNC_WORDS,), dtype=torch.int32, device=dev)
    ref = _run(_hip, dev, x, pos, heads, D, S, ns, H, E, fused=False)
    _run(_hip, dev, x, pos, heads, D, S, ns, H, E, fused=True, sync=sync, timeout_us=0)
    assert int(sync[0].item()) & 1, "no wait reported a timeout"
    _hip.call("lemoq_sync_reset", _hip.ptr(sync), _hip.stream_of(dev))
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(sync)) == 0
    got = _run(_hip, dev, x, pos, heads, D, S, ns, H, E, fused=True, sync=sync)
    assert int(sync[0].item()) == 0
    _bitwise(ref, got, "after reset")


def test_attn_layer_rejects_before_launch(dev):
    from lemoq import _hip

    lib = _hip.load()
    assert int(lib.lemoq_attn_layer_check(16, 64, 16, 2048, 128, 64)) != 0   # head_dim 64
    assert int(lib.lemoq_attn_layer_check(6, 128, 16, 2048, 128, 64)) != 0   # heads % 4
    assert int(lib.lemoq_attn_layer_check(16, 128, 65, 2048, 128, 64)) != 0  # > 64 splits
    assert int(lib.lemoq_attn_layer_check(16, 128, 16, 3072, 128, 64)) != 0  # hidden
    assert int(lib.lemoq_attn_layer_check(4, 128, 1, 2048, 128, 64)) != 0    # 16 router blocks > 4 workgroups
    assert int(lib.lemoq_attn_layer_check(16, 128, 16, 2048, 128, 64)) == 0
