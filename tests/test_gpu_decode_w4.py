"""GPU parity of the decode step on 4-bit weights and with an fp16 lm_head: the
reference's w4a16 cell (``--bit-width w4a16``: attention and experts as 4-bit
symmetric RTN codes, group 128, router and lm_head in fp16,
benchmarks/runner.py:393-412,451-482), run through ``lemoq_olmoe_decode_step``
with ``weight_bits`` 4 / ``lm_f16``.

- The two launches the 4-bit layer adds: the o_proj GEMV with the residual add
  (``lemoq_gemv_q_residual``) equals ``lemoq_gemv_q`` followed by torch's fp16
  add, bit for bit, in place or not; the routed 4-bit gate/up equals
  ``lemoq_route_topk`` followed by ``lemoq_moe_gate_up_w4`` (ids, fp16 weights
  and the activations bit for bit), ties included.
- Whole sessions against ``OracleDecoder`` on the same weights (the oracle
  unpacks the 4-bit codes, oracle.quant.unpack_4bit, and computes code * scale
  as for 8 bits; its fp16 lm_head is an fp16 F.linear), from the GPU's KV
  cache after the prompt, with the gates of the w8 step: per step logits KL <
  0.01, max |diff| within 2% of the largest logit, the greedy token equal to
  the oracle's argmax (exact fp16 ties aside); graph == eager bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from helpers import randn
from lemoq import _hip
from lemoq.model.olmoe import OLMOE_1B_7B, DecodeSession, OlmoeShape, OlmoeW8Weights
from oracle import ops
from oracle.olmoe import OracleDecoder
from test_gpu_decode import TINY, _check_steps, _kv_equal

pytestmark = pytest.mark.gpu

W4 = 2  # LEMOQ_QFMT_W4
STEPS = 32


def _q4(w, dev):
    from lemoq.quant.rtn import quantize_rtn

    q = quantize_rtn(w.to(dev), bits=4, group_size=128)
    return q["packed"], q["scale_f16"]


@pytest.mark.parametrize("M,N,K", [(1, 2048, 2048), (3, 640, 1024), (1, 6144, 2048)])
def test_gemv_q_residual_equals_gemv_then_fp16_add(M, N, K, dev):
    print("case: gemv_q_residual M %d N %d K %d" % (M, N, K), flush=True)
    P, st = _hip.ptr, _hip.stream_of(dev)
    codes, scale = _q4(randn(N, K, seed=N + K, std=0.02), dev)
    x = randn(M, K, seed=2).to(torch.float16).to(dev)
    res = randn(M, N, seed=3, std=4.0).to(torch.float16).to(dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    _hip.call("lemoq_gemv_q", P(x), M, K, P(codes), W4, P(scale), None, 0, N, K, 128, P(y), 1, st)
    ref = (y.float().cpu() + res.float().cpu()).to(torch.float16)  # torch's fp16 add: one rounding
    out = torch.empty_like(res)
    _hip.call("lemoq_gemv_q_residual", P(x), M, K, P(codes), W4, P(scale), None, 0, N, K, 128, P(res), P(out), st)
    inplace = res.clone()
    _hip.call("lemoq_gemv_q_residual", P(x), M, K, P(codes), W4, P(scale), None, 0, N, K, 128, P(inplace),
              P(inplace), st)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ref) and torch.equal(inplace.cpu(), ref)


@pytest.mark.parametrize("K", [2048, 4096])
def test_qkv_norm_gemv_gathers_the_embedding_row(K, dev):
    """lemoq_gemv_q_rmsnorm with x_row_index (layer 0 of the 4-bit step: the
    embedding row of the device token, normalised once per block): the outputs
    equal those of the same call on the row itself, bit for bit; x_copy receives
    the raw row; an index outside the table reads as a zero row (zero outputs,
    zero copy)."""
    print("case: 4-bit q|k|v GEMV with the gather, K %d" % K, flush=True)
    P, st = _hip.ptr, _hip.stream_of(dev)
    N, V = 768, 50
    codes, scale = _q4(randn(N, K, seed=K + 1, std=0.02), dev)
    embed = randn(V, K, seed=K + 2).to(torch.float16).to(dev)
    nw = (torch.rand(K, generator=torch.Generator().manual_seed(K + 3)) + 0.5).to(torch.float16).to(dev)
    for idx in (7, V - 1, V, -3):
        tok = torch.tensor([idx], dtype=torch.int64, device=dev)
        y = torch.empty(N, dtype=torch.float16, device=dev)
        copy = torch.full((K,), 7.0, dtype=torch.float16, device=dev)
        _hip.call("lemoq_gemv_q_rmsnorm", P(embed), P(tok), V, 1, K, P(nw), 1e-5, P(copy), P(codes), W4, P(scale),
                  None, 0, N, K, 128, P(y), 1, st)
        row = embed[idx].clone() if 0 <= idx < V else torch.zeros(K, dtype=torch.float16, device=dev)
        y_ref = torch.empty_like(y)
        _hip.call("lemoq_gemv_q_rmsnorm", P(row), None, 0, 1, K, P(nw), 1e-5, None, P(codes), W4, P(scale), None, 0,
                  N, K, 128, P(y_ref), 1, st)
        torch.cuda.synchronize()
        assert torch.equal(copy, row), idx
        assert torch.equal(y, y_ref), idx
        if not 0 <= idx < V:
            assert not y.any()


@pytest.mark.parametrize("E,K,F,H,norm", [(64, 8, 1024, 2048, False), (8, 2, 256, 512, True),
                                          (200, 6, 128, 1024, False)])
@pytest.mark.parametrize("ties", [False, True])
def test_routed_gate_up_w4_equals_route_then_gate_up(E, K, F, H, norm, ties, dev):
    print("case: routed gate/up w4 E %d K %d F %d H %d norm %s ties %s" % (E, K, F, H, norm, ties), flush=True)
    P, st = _hip.ptr, _hip.stream_of(dev)
    codes, scale = _q4(randn(E * 2 * F, H, seed=E + F, std=0.02), dev)
    codes, scale = codes.reshape(E, 2 * F, H // 2), scale.reshape(E, 2 * F, H // 128)
    x = randn(H, seed=11).to(torch.float16).to(dev)
    lg = randn(E, seed=12)
    if ties:  # the top values repeated: index order must decide
        lg[::3] = lg.max()
    logits = lg.to(torch.float16).to(dev)
    tw32 = torch.empty(K, dtype=torch.float32, device=dev)
    ti = torch.empty(K, dtype=torch.int64, device=dev)
    _hip.call("lemoq_route_topk", P(logits), 1, 1, E, E, K, int(norm), P(tw32), P(ti), st)
    act = torch.empty((K, F), dtype=torch.float16, device=dev)
    _hip.call("lemoq_moe_gate_up_w4", P(x), P(codes), P(scale), P(ti), K, E, F, H, 128, P(act), st)
    act2 = torch.empty_like(act)
    ti2 = torch.empty_like(ti)
    tw2 = torch.empty(K, dtype=torch.float16, device=dev)
    _hip.call("lemoq_moe_gate_up_w4_routed", P(x), P(codes), P(scale), P(logits), K, int(norm), E, F, H, 128,
              P(act2), P(ti2), P(tw2), st)
    torch.cuda.synchronize()
    assert torch.equal(ti2, ti) and torch.equal(tw2, tw32.to(torch.float16)) and torch.equal(act2, act)
    _, ri = ops.route_logits(lg.to(torch.float16).reshape(1, E), K, norm)  # the oracle's ids
    assert torch.equal(ti2.cpu(), ri.reshape(-1))


def _weights(shape, bits, lm_head, seed, dev):
    return OlmoeW8Weights.random(shape, seed=seed, device=dev, bits=bits, lm_head=lm_head)


@pytest.mark.parametrize("bits,lm_head,kv", [(4, "fp16", "int8"), (4, "fp16", "fp16"), (4, "w8", "int8"),
                                             (8, "fp16", "int8")])
def test_tiny_model_matches_oracle(bits, lm_head, kv, dev):
    """Random prompt fed through the step, then 32 greedy steps against the
    oracle from the GPU's cache; the same for 8-bit weights with the fp16
    lm_head (the 8-bit layer, the fp16 head)."""
    print("case: tiny model bits %d lm_head %s kv %s" % (bits, lm_head, kv), flush=True)
    w = _weights(TINY, bits, lm_head, 31, dev)
    ctx = 40
    prompt = torch.randint(0, TINY.vocab, (ctx,), generator=torch.Generator().manual_seed(32)).tolist()
    sess = DecodeSession(w, prompt, max_new_tokens=STEPS, kv_cache=kv)
    assert not sess.attn_output_fused  # hidden 512: merge, o_proj (+ residual), router as three launches
    assert sess.launches_per_step == 7 * TINY.layers + 2 + (bits == 4)
    seed = sess.prefill(mode="stepped")
    oracle = OracleDecoder(w.to_host(), sess.max_seq, kv=sess.kv_cpu())
    gl = []
    for _ in range(STEPS):
        sess.replay(1)
        gl.append(sess.logits_cpu())
    toks = [int(t) for t in sess.history[ctx: ctx + STEPS + 1].tolist()]
    assert toks[0] == seed
    rl = [oracle.step(toks[i], ctx + i) for i in range(STEPS)]
    _check_steps(toks, gl, rl)


@pytest.mark.parametrize("kv", ["int8", "fp16"])
def test_tiny_fused_shape_w4_matches_oracle(kv, dev):
    """Hidden 2048 and 16 heads at 2 layers: the 4-bit layer's fused attention
    output (merge + 4-bit o_proj, residual + norm + router); 32 greedy steps
    against the oracle from the GPU's cache."""
    from test_gpu_decode import TINY_FUSED

    print("case: tiny fused-shape w4a16 model, kv %s" % kv, flush=True)
    w = _weights(TINY_FUSED, 4, "fp16", 36, dev)
    ctx = 40
    prompt = torch.randint(0, TINY_FUSED.vocab, (ctx,), generator=torch.Generator().manual_seed(37)).tolist()
    sess = DecodeSession(w, prompt, max_new_tokens=STEPS, kv_cache=kv)
    assert sess.attn_output_fused and sess.launches_per_step == 6 * TINY_FUSED.layers + 2
    sess.prefill(mode="stepped")
    oracle = OracleDecoder(w.to_host(), sess.max_seq, kv=sess.kv_cpu())
    gl = []
    for _ in range(STEPS):
        sess.replay(1)
        gl.append(sess.logits_cpu())
    toks = [int(t) for t in sess.history[ctx: ctx + STEPS + 1].tolist()]
    rl = [oracle.step(toks[i], ctx + i) for i in range(STEPS)]
    _check_steps(toks, gl, rl)


@pytest.mark.parametrize("shape", ["tiny", "tiny_fused"])
def test_batched_prefill_of_4bit_weights_matches_oracle(shape, dev):
    """The batched prefill of the w4a16 cell (the prefill GEMMs on the int8
    re-encoding of the 4-bit codes, the fp16 lm_head for the last row) against
    the oracle's prefill of the same weights: last logits (KL < 0.01, max |diff|
    within 2%), the seed token (near-ties aside), every layer's KV-INT8 bytes
    (kv_rows_vs_oracle); then 8 decode steps against the oracle from the GPU's
    cache."""
    from helpers import kv_rows_vs_oracle
    from oracle.olmoe import oracle_prefill
    from test_gpu_decode import TINY_FUSED

    print("case: batched prefill, 4-bit weights, %s" % shape, flush=True)
    sh = TINY if shape == "tiny" else TINY_FUSED
    w = _weights(sh, 4, "fp16", 38, dev)
    T, steps = 48, 8
    prompt = torch.randint(0, sh.vocab, (T,), generator=torch.Generator().manual_seed(39)).tolist()
    sess = DecodeSession(w, prompt, max_new_tokens=steps)
    rows = []
    seed_tok = sess.prefill(kv_f16=rows)
    logits, kv = sess.logits_cpu(), sess.kv_cpu()
    hw = w.to_host()
    ref_rows = []
    ref, ref_kv = oracle_prefill(hw, prompt, sess.max_seq, kv_f16=ref_rows)
    r64, g64 = ref.double(), logits.double()
    p, q = torch.log_softmax(r64, -1), torch.log_softmax(g64, -1)
    kl, diff = float((p.exp() * (p - q)).sum()), float((r64 - g64).abs().max())
    print("prefill: KL %.2e, max|diff| %.3e" % (kl, diff))
    assert kl < 1e-2 and diff <= 2e-2 * float(r64.abs().max())
    if seed_tok != int(torch.argmax(r64)):
        top = torch.topk(r64, 2).values
        assert float(top[0] - top[1]) <= 2 * diff
    for li in range(sh.layers):
        kv_rows_vs_oracle("w4 prefill layer %d" % li, kv[li], rows[li], ref_kv[li], ref_rows[li], T,
                          rows_close=li == 0)
    gl = []
    for _ in range(steps):
        sess.replay(1)
        gl.append(sess.logits_cpu())
    toks = [int(t) for t in sess.history[T: T + steps + 1].tolist()]
    oracle = OracleDecoder(hw, sess.max_seq, kv=kv)
    _check_steps(toks, gl, [oracle.step(toks[i], T + i) for i in range(steps)])


def test_tiny_model_prompt_steps_match_oracle_run(dev):
    """The prompt's own steps: the GPU's stepped prefill and 8 greedy steps give
    the oracle's run() tokens from an empty cache (every prompt position through
    both implementations)."""
    print("case: tiny w4 model, oracle run from position 0", flush=True)
    w = _weights(TINY, 4, "fp16", 33, dev)
    prompt = torch.randint(0, TINY.vocab, (24,), generator=torch.Generator().manual_seed(34)).tolist()
    sess = DecodeSession(w, prompt, max_new_tokens=8)
    sess.prefill(mode="stepped")
    sess.replay(8)
    got = sess.generated()
    toks, _ = OracleDecoder(w.to_host(), sess.max_seq).run(prompt, 8)
    assert got == toks, (got, toks)


def test_olmoe_shape_w4a16_random_prompt(dev):
    """The OLMoE-1B-7B shape as the w4a16 cell (4-bit attention and experts, fp16
    lm_head, KV-INT8), a seeded random 192-token prompt fed through the step:
    graph == eager bit for bit over 4 positions, then 16 greedy steps against
    the oracle from the GPU's cache (strict argmax rule: only an exact fp16 tie
    excuses a flip)."""
    print("case: OLMoE shape w4a16, random 192-token prompt", flush=True)
    w = _weights(OLMOE_1B_7B, 4, "fp16", 41, dev)
    ctx = 192
    prompt = torch.randint(0, OLMOE_1B_7B.vocab, (ctx,), generator=torch.Generator().manual_seed(42)).tolist()
    sess = DecodeSession(w, prompt, max_new_tokens=24)
    assert sess.attn_output_fused and sess.launches_per_step == 6 * 16 + 2
    sess.prefill(mode="stepped")
    pos0, tok0 = sess.position, sess.next_token_cpu()
    kv0 = sess.kv_cpu()
    eager = [sess.decode_eager().clone() for _ in range(4)]
    kv_e = sess.kv_cpu()
    sess.set_position(pos0, tok0)
    graph = [sess.replay(1).clone() for _ in range(4)]
    assert all(torch.equal(a, b) for a, b in zip(eager, graph))
    assert _kv_equal(kv_e, sess.kv_cpu())
    sess.set_position(pos0, tok0)
    oracle = OracleDecoder(w.to_host(), sess.max_seq, kv=kv0)
    gl = []
    for _ in range(16):
        sess.replay(1)
        gl.append(sess.logits_cpu())
    toks = [tok0] + [int(t) for t in sess.history[pos0 + 1: pos0 + 17].tolist()]
    rl = [oracle.step(toks[i], pos0 + i) for i in range(16)]
    _check_steps(toks, gl, rl, strict=True)


def test_session_rejects_mismatched_weights(dev):
    """A 4-bit weight set with group 64 is refused at construction of the
    weights; the step refuses what its 4-bit rules exclude before any launch."""
    bad = OlmoeShape(**{**TINY.__dict__, "group_size": 16})
    with pytest.raises(ValueError):
        OlmoeW8Weights.random(bad, seed=1, device=dev, bits=4)
    w = _weights(TINY, 4, "fp16", 35, dev)
    w.bits = 5
    with pytest.raises(ValueError):
        DecodeSession(w, [1, 2, 3], max_new_tokens=2)
