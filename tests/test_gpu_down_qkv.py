"""GPU tests of lemoq_moe_down_qkv_w8: the down projection of layer L and the
input RMSNorm + packed q|k|v GEMV of layer L+1 as one launch.

The fused launch must give exactly the bits of the two launches it replaces
(lemoq_moe_down_w8 with the residual, then lemoq_gemv_w8_fused with the norm
prologue), whose arithmetic the operator tests pin against the oracle.  The
workgroups hand h to each other through a buffer whose words carry a flag
unique to the launch (from a launch counter the launch advances), so calls
in a row reuse it without clearing; a forced give-up (zero time limit) must
record the status bit and still drain the grid.  A whole decode session with
the fused launch must match the default session bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from lemoq import _hip
from lemoq.model.olmoe import DecodeSession, OlmoeShape, OlmoeW8Weights

pytestmark = pytest.mark.gpu

H, F, E, TOPK, NQKV, G = 2048, 1024, 16, 8, 6144, 128


def _q8(w: torch.Tensor, dev):
    """Symmetric per-group-128 int8 codes and fp16 scales of an fp32 (N, K) matrix."""
    N, K = w.shape
    g = w.reshape(N, K // G, G)
    scale = (g.abs().amax(-1) / 127.0).clamp_min(1e-8).half()
    codes = torch.clamp(torch.round(g / scale.float().unsqueeze(-1)), -127, 127).to(torch.int8)
    return codes.reshape(N, K).contiguous().to(dev), scale.contiguous().to(dev)


def _inputs(dev, seed=0):
    gen = torch.Generator().manual_seed(seed)
    dn = torch.randn((E * H, F), generator=gen) * 0.02
    dn_c, dn_s = _q8(dn, dev)
    qkv = torch.randn((NQKV, H), generator=gen) * 0.02
    qkv_c, qkv_s = _q8(qkv, dev)
    act = (torch.randn((TOPK, F), generator=gen) * 0.5).half().to(dev)
    ids = torch.randperm(E, generator=gen)[:TOPK].to(torch.int64).to(dev)
    top_w = torch.softmax(torch.randn(TOPK, generator=gen), 0).half().to(dev)
    resid = torch.randn(H, generator=gen).half().to(dev)
    norm_w = (0.5 + torch.rand(H, generator=gen)).half().to(dev)
    return dict(dn_c=dn_c, dn_s=dn_s, qkv_c=qkv_c, qkv_s=qkv_s, act=act, ids=ids, top_w=top_w, resid=resid,
                norm_w=norm_w)


def _reference(x, dev, eps=1e-5):
    P = _hip.ptr
    st = _hip.stream_of(dev)
    h = torch.empty(H, dtype=torch.float16, device=dev)
    q = torch.empty(NQKV, dtype=torch.float16, device=dev)
    _hip.call("lemoq_moe_down_w8", P(x["act"]), P(x["dn_c"]), P(x["dn_s"]), P(x["ids"]), P(x["top_w"]), TOPK, E, H,
              F, G, P(x["resid"]), P(h), st)
    _hip.call("lemoq_gemv_w8_fused", P(h), None, 0, P(x["norm_w"]), eps, None, P(x["qkv_c"]), P(x["qkv_s"]), NQKV,
              H, G, None, P(q), st)
    torch.cuda.synchronize(dev)
    return h, q


def _fused(x, dev, ll, sync, timeout_us=200_000, eps=1e-5):
    P = _hip.ptr
    h = torch.full((H,), float("nan"), dtype=torch.float16, device=dev)
    q = torch.full((NQKV,), float("nan"), dtype=torch.float16, device=dev)
    _hip.call("lemoq_moe_down_qkv_w8", P(x["act"]), P(x["dn_c"]), P(x["dn_s"]), P(x["ids"]), P(x["top_w"]), TOPK,
              E, H, F, G, P(x["resid"]), P(h), P(x["norm_w"]), eps, P(x["qkv_c"]), P(x["qkv_s"]), NQKV, P(q),
              P(ll), P(sync), timeout_us, _hip.stream_of(dev))
    torch.cuda.synchronize(dev)
    return h, q


def _buffers(dev):
    # the hand-off buffer (H / 2 64-bit words, 256-byte aligned) and the sync
    # words (status, launch counter), zeroed together
    ws = torch.zeros(H // 2 + 32, dtype=torch.int64, device=dev)
    assert ws.data_ptr() % 256 == 0
    return ws[: H // 2], ws[H // 2: H // 2 + 1].view(torch.int32)


def test_check_covers_the_olmoe_shape(dev):
    lib = _hip.load()
    assert int(lib.lemoq_moe_down_qkv_check(TOPK, H, F, G, NQKV)) == 0
    # outside the covered shapes: the two launches must be used
    assert int(lib.lemoq_moe_down_qkv_check(TOPK, 4096, F, G, NQKV)) == -3
    assert int(lib.lemoq_moe_down_qkv_check(16, H, F, G, NQKV)) == -3
    assert int(lib.lemoq_moe_down_qkv_check(TOPK, H, F, G, 6000)) == -3


def test_fused_equals_two_launches_bitwise(dev):
    print("case: down_qkv fused vs down + qkv, OLMoE shape, three calls on one buffer", flush=True)
    ll, sync = _buffers(dev)
    for call, seed in enumerate((1, 2, 1)):
        x = _inputs(dev, seed=seed)
        h_ref, q_ref = _reference(x, dev)
        h, q = _fused(x, dev, ll, sync)
        st, gen = sync.tolist()
        assert st == 0
        assert gen == call + 1, "the launch counter advances once per launch"
        assert torch.equal(h.view(torch.int16), h_ref.view(torch.int16)), call
        assert torch.equal(q.view(torch.int16), q_ref.view(torch.int16)), call
        assert int((ll >> 32).ne(2 * call + 1).sum()) == 0, "every word carries this launch's flag"


def test_stale_words_of_an_earlier_launch_are_not_taken(dev):
    """Words left by a launch with other inputs must not stand in for this
    launch's: after a call on seed 3, a call on seed 4 on the same buffer equals
    the two launches on seed 4."""
    print("case: down_qkv, stale hand-off words from another launch", flush=True)
    ll, sync = _buffers(dev)
    _fused(_inputs(dev, seed=3), dev, ll, sync)
    x = _inputs(dev, seed=4)
    h_ref, q_ref = _reference(x, dev)
    h, q = _fused(x, dev, ll, sync)
    assert sync.tolist() == [0, 2]
    assert torch.equal(h.view(torch.int16), h_ref.view(torch.int16))
    assert torch.equal(q.view(torch.int16), q_ref.view(torch.int16))


def test_invalid_expert_id_gives_zero_contribution(dev):
    print("case: down_qkv with an out-of-range expert id", flush=True)
    x = _inputs(dev, seed=3)
    x["ids"][3] = E + 5
    h_ref, q_ref = _reference(x, dev)
    ll, sync = _buffers(dev)
    h, q = _fused(x, dev, ll, sync)
    assert int(sync[0].item()) == 0
    assert torch.equal(h.view(torch.int16), h_ref.view(torch.int16))
    assert torch.equal(q.view(torch.int16), q_ref.view(torch.int16))


def test_forced_give_up_sets_status_and_drains(dev):
    print("case: down_qkv with a zero time limit (forced give-up)", flush=True)
    x = _inputs(dev, seed=4)
    ll, sync = _buffers(dev)
    h, _ = _fused(x, dev, ll, sync, timeout_us=0)
    # the down half never waits: h is still exact
    h_ref, _ = _reference(x, dev)
    assert torch.equal(h.view(torch.int16), h_ref.view(torch.int16))
    st, gen = sync.tolist()
    assert st & _hip.SYNC_TIMEOUT_BIT, "no workgroup gave up at a zero time limit"
    assert gen == 1


def test_rejects_bad_arguments(dev):
    x = _inputs(dev, seed=5)
    ll, sync = _buffers(dev)
    P = _hip.ptr
    h = torch.empty(H, dtype=torch.float16, device=dev)
    q = torch.empty(NQKV, dtype=torch.float16, device=dev)
    lib = _hip.load()
    args = [P(x["act"]), P(x["dn_c"]), P(x["dn_s"]), P(x["ids"]), P(x["top_w"]), TOPK, E, H, F, G, P(x["resid"]),
            P(h), P(x["norm_w"]), 1e-5, P(x["qkv_c"]), P(x["qkv_s"]), NQKV, P(q), P(ll), P(sync), 1000,
            _hip.stream_of(dev)]
    bad = list(args)
    bad[18] = P(ll) + 8  # hand-off buffer not 256-byte aligned
    assert int(lib.lemoq_moe_down_qkv_w8(*bad)) == -4
    bad = list(args)
    bad[19] = P(ll) + 64  # sync words inside the buffer
    assert int(lib.lemoq_moe_down_qkv_w8(*bad)) == -2
    bad = list(args)
    bad[20] = -1
    assert int(lib.lemoq_moe_down_qkv_w8(*bad)) == -2
    bad = list(args)
    bad[19] = None
    assert int(lib.lemoq_moe_down_qkv_w8(*bad)) == -1
    assert sync.tolist() == [0, 0]  # nothing ran


# hidden 2048 / ffn 1024 / top_k 8: the fused launch's shape; 4 layers (3 fused launches per step)
DQ_SHAPE = OlmoeShape(hidden=2048, heads=16, head_dim=128, layers=4, num_experts=16, top_k=8, ffn=1024,
                      vocab=2048)


@pytest.mark.parametrize("graph", [False, True])
def test_session_with_fused_launch_matches_default_bitwise(graph, dev):
    print("case: DecodeSession down_qkv_fused vs default, 4 layers, graph=%s" % graph, flush=True)
    w = OlmoeW8Weights.random(DQ_SHAPE, seed=11, device=dev)
    prompt = torch.randint(0, DQ_SHAPE.vocab, (48,), generator=torch.Generator().manual_seed(5)).tolist()
    out = []
    for fused in (False, True):
        sess = DecodeSession(w, prompt, max_new_tokens=12, down_qkv_fused=fused)
        assert sess.down_qkv_fused == fused
        assert sess.launches_per_step == 6 * 4 + 2 - (3 if fused else 0)
        if graph:
            sess.capture()
        sess.prefill()
        logits = []
        for _ in range(10):
            if graph:
                sess.replay(1)
            else:
                sess.decode_eager()
            logits.append(sess.logits_cpu())
        sess.check_sync_status()
        out.append((sess.generated(), logits))
        del sess
    (t0, l0), (t1, l1) = out
    assert t0 == t1
    for a, b in zip(l0, l1):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
