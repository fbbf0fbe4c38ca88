"""The gate and statistics helpers of ``lemoq.model.graph_session`` on the CPU:
``compare_logits`` (mean KL and top-1 agreement, the reference's
``benchmarks/cudagraph.py:298-325``), the gate predicate (``:328-339``) and
``summarize`` (linear-interpolation percentiles, ``benchmarks/timing.py:26-69``)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from lemoq.model.graph_session import compare_logits, graph_correctness_passed, summarize


def test_compare_logits_identical_and_shifted():
    a = [torch.randn(50, generator=torch.Generator().manual_seed(i)) for i in range(4)]
    r = compare_logits(a, [x.clone() for x in a])
    assert r == {"kl": 0.0, "top1_agreement": 1.0}
    # adding a constant changes nothing (softmax), a swapped top-1 changes agreement
    r = compare_logits(a, [x + 3.0 for x in a])
    assert r["kl"] < 1e-6 and r["top1_agreement"] == 1.0  # fp32 rounding of the shift only
    b = [x.clone() for x in a]
    i = int(torch.argmax(b[0]))
    b[0][i] = -100.0
    r = compare_logits(a, b)
    assert r["top1_agreement"] == 0.75 and r["kl"] > 0.0
    # KL by hand for one step
    p, q = torch.log_softmax(a[0], -1), torch.log_softmax(b[0], -1)
    assert math.isclose(compare_logits(a[:1], b[:1])["kl"], float((p.exp() * (p - q)).sum()), rel_tol=1e-6)
    with pytest.raises(ValueError):
        compare_logits(a, a[:2])


def test_gate_predicate():
    ok = {"kl": 0.0, "top1_agreement": 1.0, "seed_token_match": True, "token_sequence_match": True}
    assert graph_correctness_passed(ok)
    for k, v in (("kl", 2e-5), ("kl", float("nan")), ("top1_agreement", 0.99), ("seed_token_match", False),
                 ("token_sequence_match", False), ("kl", None)):
        assert not graph_correctness_passed({**ok, k: v}), (k, v)


def test_nonfinite_logits_fail_the_gate():
    """A NaN or infinite candidate logit gives a non-finite KL, which the gate
    refuses (the reference's tests/test_cudagraph.py:328-342)."""
    a = [torch.randn(40, generator=torch.Generator().manual_seed(10 + i)) for i in range(3)]
    for bad in (float("nan"), float("inf")):
        b = [x.clone() for x in a]
        b[1][7] = bad
        r = compare_logits(a, b)
        assert not math.isfinite(r["kl"])
        assert not graph_correctness_passed({**r, "seed_token_match": True, "token_sequence_match": True})
    # mixed dtypes and shapes of one step's logits are compared as fp32 rows
    r = compare_logits([x.reshape(1, 1, -1).half() for x in a], [x.double() for x in a])
    assert r["top1_agreement"] == 1.0 and 0.0 <= r["kl"] < 1e-6


def test_summarize_matches_numpy_percentiles():
    xs = [0.5, 0.51, 0.49, 0.52, 0.50, 0.7]
    s = summarize(xs)
    assert s["n"] == 6 and s["p50"] == pytest.approx(np.percentile(xs, 50))
    assert s["p99"] == pytest.approx(np.percentile(xs, 99)) and s["min"] == 0.49 and s["max"] == 0.7
    assert s["cov"] == pytest.approx(np.std(xs) / np.mean(xs))
    with pytest.raises(ValueError):
        summarize([])
