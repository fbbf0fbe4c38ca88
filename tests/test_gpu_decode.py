"""GPU parity of the whole decode step (A17/A18) against the CPU oracle.

The BASELINE gates for the full step: identical greedy tokens over 32 steps
and logits KL < 0.01, here per step, plus the reference session's own gate
that the captured graph and the eager step agree exactly
(benchmarks/cudagraph.py:298-339 of LeanMoE-Quant: KL 0, identical tokens).
The oracle decodes from the GPU's KV-INT8 cache after prefill (the cache
bytes themselves are pinned bit-exactly by the KV write tests), so every
compared step runs the same inputs through both implementations.
"""

from __future__ import annotations

import pytest
import torch

from lemoq.model.olmoe import OLMOE_1B_7B, DecodeSession, OlmoeShape, OlmoeW8Weights
from oracle.olmoe import OracleDecoder

pytestmark = pytest.mark.gpu

TINY = OlmoeShape(hidden=512, heads=4, head_dim=128, layers=2, num_experts=8, top_k=2, ffn=256, vocab=1024)
# hidden 2048, 16 heads: the step takes the fused attention-output path (merge + o_proj over
# 4-head groups, residual in the router launch); TINY takes the three-launch path.
TINY_FUSED = OlmoeShape(hidden=2048, heads=16, head_dim=128, layers=2, num_experts=8, top_k=2, ffn=256,
                        vocab=1024)
# 8 heads (attention width 1024 != hidden 2048: two partial rows) and, at a
# 1200-slot cache, more than 16 splits per head (the 64-split merge instance)
NARROW_FUSED = OlmoeShape(hidden=2048, heads=8, head_dim=128, layers=2, num_experts=8, top_k=2, ffn=256,
                          vocab=1024)


def _kl(p_logits, q_logits) -> float:
    p = torch.log_softmax(p_logits.double(), -1)
    q = torch.log_softmax(q_logits.double(), -1)
    return float((p.exp() * (p - q)).sum())


def _margin(logits) -> float:
    top = torch.topk(logits.float(), 2).values
    return float(top[0] - top[1])


def _teacher_forced(shape, prompt, steps, seed, dev, *, norm_topk_prob=False):
    """GPU decodes greedily; the oracle processes the GPU's token at every step
    (from the GPU's KV cache after prefill) so each step compares the same input.
    Returns per-step (gpu logits, oracle logits) and the GPU token sequence."""
    if norm_topk_prob:
        shape = OlmoeShape(**{**shape.__dict__, "norm_topk_prob": True})
    w = OlmoeW8Weights.random(shape, seed=seed, device=dev)
    sess = DecodeSession(w, prompt, max_new_tokens=steps, num_splits=None)
    sess.prefill()
    kv = sess.kv_cpu()
    gpu_logits = []
    for _ in range(steps):
        sess.replay(1)
        gpu_logits.append(sess.logits_cpu())
    toks = [int(t) for t in sess.history[len(prompt) - 1: len(prompt) + steps].tolist()]
    oracle = OracleDecoder(w.to_host(), sess.max_seq, kv=kv)
    ref_logits = [oracle.step(toks[i + 1], len(prompt) + i) for i in range(steps)]
    return toks, gpu_logits, ref_logits


def _check_steps(toks, gl, rl, *, rel=2e-2):
    """Per step: logits KL < 0.01 (the BASELINE gate for the full step), max
    |diff| below ``rel`` of the largest logit, and the GPU's greedy token is the
    oracle's argmax unless the oracle's own top-1/top-2 margin is below twice
    the measured logit difference (a near-tie, printed)."""
    flips = []
    for i, (a, b) in enumerate(zip(gl, rl)):
        diff = float((a.float() - b.float()).abs().max())
        scale = float(b.float().abs().max())
        kl = _kl(b, a)
        m = _margin(b)
        ga, ra = int(torch.argmax(a.float())), int(torch.argmax(b.float()))
        print("step %2d tok %6d diff %.2e |max| %.2e kl %.1e margin %.2e argmax gpu %d oracle %d"
              % (i, toks[i + 2] if i + 2 < len(toks) else -1, diff, scale, kl, m, ga, ra))
        assert diff <= rel * scale, (i, diff, scale)
        assert kl < 1e-2, (i, kl)
        if ga != ra:
            flips.append((i, m, diff))
            assert m <= 2 * diff, (i, m, diff)
    return flips


@pytest.mark.parametrize("norm", [False, True])
def test_tiny_model_32_steps_match_oracle(norm, dev):
    print("case: tiny model, 32 steps, norm_topk_prob=%s" % norm, flush=True)
    toks, gl, rl = _teacher_forced(TINY, [1] * 16, 32, 3, dev, norm_topk_prob=norm)
    _check_steps(toks, gl, rl)


@pytest.mark.parametrize("shape,ctx,norm", [("tiny", 40, False), ("tiny", 40, True), ("narrow", 1200, False)])
def test_fused_path_model_32_steps_match_oracle(shape, ctx, norm, dev):
    print("case: %s fused-path test model, ctx %d, 32 steps, norm_topk_prob=%s" % (shape, ctx, norm), flush=True)
    sh = TINY_FUSED if shape == "tiny" else NARROW_FUSED
    w = OlmoeW8Weights.random(sh, seed=4, device=dev)
    probe = DecodeSession(w, [1] * ctx, max_new_tokens=32)
    assert probe.attn_output_fused
    if shape == "narrow":
        assert probe.num_splits > 16, probe.num_splits
    del probe
    toks, gl, rl = _teacher_forced(sh, [1] * ctx, 32, 4, dev, norm_topk_prob=norm)
    _check_steps(toks, gl, rl)


def test_olmoe_shape_32_greedy_steps_match_oracle(dev):
    """Full OLMoE-1B-7B shape (16 layers, 64 experts top-8, vocab 50304) at ctx 256:
    every step's logits agree (KL < 0.01) and the greedy token equals the
    oracle's argmax except at near-ties (random-init logits have top-1/top-2
    margins down to one fp16 ulp; such steps are printed).  A step where the
    oracle's top two fp16 logits are exactly equal (margin 0) is decided by
    index order alone, so the reference is indifferent between the two tokens:
    such flips are listed but not counted.  At most 2 flips at a non-zero
    margin are allowed, each within twice the measured logit difference."""
    print("case: OLMoE shape, ctx 256, 32 steps", flush=True)
    toks, gl, rl = _teacher_forced(OLMOE_1B_7B, [1] * 256, 32, 0, dev)
    flips = _check_steps(toks, gl, rl)
    exact_ties = [f for f in flips if f[1] == 0.0]
    counted = [f for f in flips if f[1] != 0.0]
    print("near-tie flips:", counted, "flips at exact fp16 ties:", exact_ties)
    assert len(counted) <= 2, flips


def test_graph_replay_equals_eager_step_bitwise(dev):
    print("case: graph vs eager", flush=True)
    w = OlmoeW8Weights.random(TINY, seed=5, device=dev)
    sess = DecodeSession(w, [1] * 8, max_new_tokens=4, num_splits=4)
    sess.prefill()
    p = sess.position
    tok = int(sess.token.item())
    sess.replay(1)
    g_logits = sess.logits_cpu()
    g_next = int(sess.token.item())
    sess.set_position(p, tok)
    sess.decode_eager()
    e_logits = sess.logits_cpu()
    assert torch.equal(g_logits, e_logits)
    assert int(sess.token.item()) == g_next
    # replaying the same position again is deterministic
    sess.set_position(p, tok)
    sess.replay(1)
    assert torch.equal(sess.logits_cpu(), g_logits)


def test_prompt_tokens_are_fed_then_greedy_takes_over(dev):
    print("case: prompt feed", flush=True)
    w = OlmoeW8Weights.random(TINY, seed=6, device=dev)
    prompt = [5, 17, 300, 2, 999, 42]
    sess = DecodeSession(w, prompt, max_new_tokens=3, num_splits=2)
    sess.prefill(mode="stepped")  # the oracle's run() steps the prompt too
    hist = sess.history[: len(prompt)].tolist()
    assert hist == prompt
    oracle = OracleDecoder(w.to_host(), sess.max_seq)
    tokens, _ = oracle.run(prompt, 3)
    sess.replay(3)
    assert sess.generated() == tokens


def test_fused_attention_output_path_matches_three_launches(dev):
    """At the OLMoE shape the step runs merge + o_proj as one launch and the
    residual add in the router launch (lemoq_attn_merge_o_proj_w8,
    lemoq_router_logits_resid).  With o_part unset the same step runs
    lemoq_attn_merge, the o_proj GEMV and lemoq_router_logits.  Both orders of
    the o_proj fp32 sum must give the same step to fp16 rounding: per step
    logits KL < 1e-4 and the same greedy token unless the top-2 margin is
    below twice the logit difference."""
    print("case: fused vs three-launch attention output, OLMoE shape, 4 layers", flush=True)
    shape = OlmoeShape(**{**OLMOE_1B_7B.__dict__, "layers": 4})
    w = OlmoeW8Weights.random(shape, seed=11, device=dev)
    sess = DecodeSession(w, [3] * 200, max_new_tokens=8, num_splits=None)
    sess.prefill()
    o_part = sess._step.o_part
    assert o_part
    for _ in range(4):
        p, tok = sess.position, int(sess.token.item())
        sess._step.o_part = None
        sess.decode_eager()
        ref = sess.logits_cpu()
        sess._step.o_part = o_part
        sess.set_position(p, tok)
        sess.decode_eager()
        got = sess.logits_cpu()
        diff = float((got.float() - ref.float()).abs().max())
        kl = _kl(ref, got)
        print("pos %d diff %.2e kl %.1e margin %.2e" % (p, diff, kl, _margin(ref)))
        assert kl < 1e-4, kl
        if int(torch.argmax(got.float())) != int(torch.argmax(ref.float())):
            assert _margin(ref) <= 2 * diff
