"""GPU parity of the one-launch MoE of a decoder layer (lemoq_moe_layer_w8)
against the two launches it replaces: lemoq_moe_gate_up_w8_routed ->
lemoq_moe_down_w8 with the residual (themselves pinned to the oracle in
test_gpu_ops.py and test_gpu_decode.py).

The fused launch's workgroups route the token themselves, hand the SiLU
activations and the per-slot down partials to each other inside the launch
(coherent stores, counters, bounded waits) and keep the two launches'
arithmetic, so the output row, the activations and the routing (ids and fp16
weights) must be equal BIT FOR BIT, also when logits tie exactly and with
norm_topk_prob.  The sync workspace must be zero again after every successful
launch.  Failure handling is forced from the host: with a time limit of 0 the
waits give up, the status word carries LEMOQ_SYNC_TIMEOUT_BIT and the launch
completes; after lemoq_sync_reset the next launch is exact again.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

H, F, E, K, G128 = 2048, 1024, 64, 8, 128


@pytest.fixture(scope="module")
def experts(dev):
    from lemoq.model.olmoe import OlmoeShape, OlmoeW8Weights

    shape = OlmoeShape(layers=1, vocab=256)
    w = OlmoeW8Weights.random(shape, seed=21, device=dev)
    return w.layers[0]


def _run(L, x, logits, resid, norm, *, fused, sync=None, timeout_us=200_000):
    from lemoq import _hip

    dev = x.device
    P, st = _hip.ptr, _hip.stream_of(dev)
    act = torch.full((K, F), float("nan"), dtype=torch.float16, device=dev)
    out = torch.full((H,), float("nan"), dtype=torch.float16, device=dev)
    ti = torch.full((K,), -1, dtype=torch.int64, device=dev)
    tw = torch.full((K,), float("nan"), dtype=torch.float16, device=dev)
    if fused:
        ypart = torch.full((K, H), float("nan"), dtype=torch.float32, device=dev)
        _hip.call("lemoq_moe_layer_w8", P(x), P(L.gu_codes), P(L.gu_scale), P(L.dn_codes), P(L.dn_scale), P(logits),
                  K, int(norm), E, F, H, G128, P(act), P(ypart), P(resid), P(out), P(ti), P(tw), P(sync), timeout_us,
                  st)
    else:
        _hip.call("lemoq_moe_gate_up_w8_routed", P(x), P(L.gu_codes), P(L.gu_scale), P(logits), K, int(norm), E, F,
                  H, G128, P(act), P(ti), P(tw), st)
        _hip.call("lemoq_moe_down_w8", P(act), P(L.dn_codes), P(L.dn_scale), P(ti), P(tw), K, E, H, F, G128,
                  P(resid), P(out), st)
    torch.cuda.synchronize()
    return {"out": out.cpu(), "act": act.cpu(), "ti": ti.cpu(), "tw": tw.cpu()}


def _bitwise(a, b, what):
    for n in a:
        x, y = a[n], b[n]
        if x.dtype == torch.float16:
            x, y = x.view(torch.int16), y.view(torch.int16)
        assert torch.equal(x, y), "%s: %s differs" % (what, n)


def _inputs(seed, dev, ties=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((H,), generator=g).to(torch.float16).to(dev)
    logits = (torch.randn((E,), generator=g) * 2).to(torch.float16)
    if ties:  # exact fp16 ties across the top-k boundary and inside it
        logits[3] = logits[40] = logits[9] = float(logits.max()) + 0.5
        logits[17] = logits[60] = float(torch.sort(logits, descending=True).values[8])
    resid = torch.randn((H,), generator=g).to(torch.float16).to(dev)
    return x, logits.to(dev), resid


@pytest.mark.parametrize("seed,norm,ties", [(1, False, False), (2, True, False), (3, False, True), (4, True, True)])
def test_moe_layer_equals_two_launches_bitwise(seed, norm, ties, experts, dev):
    from lemoq import _hip

    print("case: moe_layer seed=%d norm=%s ties=%s" % (seed, norm, ties), flush=True)
    assert int(_hip.load().lemoq_moe_layer_check(K, E, F, H, G128)) == 0
    x, logits, resid = _inputs(seed, dev, ties)
    sync = torch.zeros((_hip.SYNC_WORDS,), dtype=torch.int32, device=dev)
    ref = _run(experts, x, logits, resid, norm, fused=False)
    for rep in range(2):
        got = _run(experts, x, logits, resid, norm, fused=True, sync=sync)
        assert int(sync[0].item()) == 0
        assert int(torch.count_nonzero(sync)) == 0, "sync workspace not returned to zero"
        _bitwise(ref, got, "rep %d" % rep)


def test_moe_layer_forced_timeout_completes_and_reports(experts, dev):
    from lemoq import _hip

    print("case: moe_layer forced timeout", flush=True)
    x, logits, resid = _inputs(5, dev)
    sync = torch.zeros((_hip.SYNC_WORDS,), dtype=torch.int32, device=dev)
    ref = _run(experts, x, logits, resid, False, fused=False)
    _run(experts, x, logits, resid, False, fused=True, sync=sync, timeout_us=0)
    assert int(sync[0].item()) & 1, "no wait reported a timeout"
    _hip.call("lemoq_sync_reset", _hip.ptr(sync), _hip.stream_of(dev))
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(sync)) == 0
    got = _run(experts, x, logits, resid, False, fused=True, sync=sync)
    assert int(sync[0].item()) == 0
    _bitwise(ref, got, "after reset")


def test_moe_layer_rejects_uncovered_shapes(dev):
    from lemoq import _hip

    lib = _hip.load()
    assert int(lib.lemoq_moe_layer_check(8, 64, 1024, 2048, 128)) == 0
    assert int(lib.lemoq_moe_layer_check(8, 128, 1024, 2048, 128)) != 0  # E > 64
    assert int(lib.lemoq_moe_layer_check(8, 64, 512, 2048, 128)) != 0   # ffn
    assert int(lib.lemoq_moe_layer_check(8, 64, 1024, 4096, 128)) != 0  # hidden
    assert int(lib.lemoq_moe_layer_check(17, 64, 1024, 2048, 128)) != 0  # top_k
