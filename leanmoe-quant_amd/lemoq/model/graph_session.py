"""Gate and timing helpers around a captured decode session.

The reference's session module carries, beside ``StaticCacheDecodeSession``,
the graph-against-eager correctness gate and the repeated step timing that
every measured cell goes through (``benchmarks/cudagraph.py:298-339,420-495``,
statistics ``benchmarks/timing.py:26-69``).  These are the same checks and
the same report keys over ``lemoq.model.olmoe.DecodeSession``:

* ``compare_logits`` / ``graph_correctness_passed`` — mean per-step KL(ref ||
  candidate) and top-1 agreement; the gate is KL <= 1e-5, top-1 agreement 1.0,
  the same seed token and the same token sequence.
* ``graph_correctness(session, steps)`` — from the session's prefilled state,
  ``steps`` eager steps, then the same steps as graph replays from the same
  state; the report that gate reads (this build's step is one native launch
  sequence, so the two are expected to agree bit for bit: ``bitwise``).
* ``measure_graph_gap(session, warmup, timed, repeats)`` — each repeat starts
  from the same prefilled state, replays ``warmup`` steps untimed, restores
  the state, then times ``timed`` replays with host wall clock and device
  events; device busy time is the event time (the step is one graph of
  ``launches_per_step`` kernels with no host work inside).
* ``summarize`` — the reference's distribution report (linear-interpolation
  percentiles, numpy's default).
"""

from __future__ import annotations

import math
import time
from typing import Any

__all__ = ["compare_logits", "graph_correctness", "graph_correctness_passed", "measure_graph_gap", "summarize"]

MIN_WARMUP = 5
MIN_TIMED = 20


def summarize(samples: Any) -> dict[str, Any]:
    """n, mean, stddev (population), min, max, p5, p50, p95, p99, coefficient of variation."""
    import numpy as np  # noqa: PLC0415

    xs = np.asarray([float(v) for v in samples], dtype=np.float64)
    if xs.size == 0:
        raise ValueError("empty sample")
    mean, sd = float(xs.mean()), float(xs.std())
    p = np.percentile(xs, [5, 50, 95, 99])
    return {"n": int(xs.size), "mean": mean, "stddev": sd, "min": float(xs.min()), "max": float(xs.max()),
            "p5": float(p[0]), "p50": float(p[1]), "p95": float(p[2]), "p99": float(p[3]),
            "cov": sd / mean if mean else 0.0, "samples": xs.tolist()}


def compare_logits(reference: list, candidate: list) -> dict[str, float]:
    """Mean over steps of KL(softmax(ref) || softmax(cand)) and the share of steps
    whose argmax agrees; both lists hold one logits vector per step (any device)."""
    import torch  # noqa: PLC0415

    if len(reference) != len(candidate) or not reference:
        raise ValueError("reference and candidate need the same non-empty number of steps")

    def rows(xs: list) -> Any:
        return torch.cat([x.detach().reshape(1, -1).to(device="cpu", dtype=torch.float32) for x in xs])

    ref, got = rows(reference), rows(candidate)
    lp, lq = torch.log_softmax(ref, -1), torch.log_softmax(got, -1)
    kl = float((lp.exp() * (lp - lq)).sum(-1).mean())
    agree = float((ref.argmax(-1) == got.argmax(-1)).float().mean())
    return {"kl": max(kl, 0.0), "top1_agreement": agree}


def graph_correctness_passed(report: dict[str, Any]) -> bool:
    """The gate every measured cell must pass: KL <= 1e-5, top-1 agreement 1.0,
    the same seed token and the same token sequence."""
    kl = report.get("kl")
    return bool(kl is not None and math.isfinite(float(kl)) and 0.0 <= float(kl) <= 1e-5
                and report.get("top1_agreement") == 1.0 and report.get("seed_token_match") is True
                and report.get("token_sequence_match") is True)


def _state(session: Any) -> tuple[int, int]:
    return session.position, int(session.token.item())


def graph_correctness(session: Any, steps: int = 8) -> dict[str, Any]:
    """Eager steps against graph replays from the session's current (prefilled)
    state; the session is left in that state.  Needs ``steps`` free cache slots."""
    import torch  # noqa: PLC0415

    if session.graph is None:
        session.capture()
    pos0, tok0 = _state(session)
    eager, eager_toks = [], []
    for _ in range(int(steps)):
        eager.append(session.decode_eager().detach().clone())
        eager_toks.append(int(session.token.item()))
    session.set_position(pos0, tok0)
    graph, graph_toks = [], []
    for _ in range(int(steps)):
        graph.append(session.replay(1).detach().clone())
        graph_toks.append(int(session.token.item()))
    session.set_position(pos0, tok0)
    report = compare_logits(eager, graph)
    report.update({
        "steps": int(steps),
        "seed_token_match": True,  # both runs start from the one prefilled token
        "seed_token": tok0,
        "token_sequence_match": eager_toks == graph_toks,
        "bitwise": all(torch.equal(a, b) for a, b in zip(eager, graph)),
    })
    report["passed"] = graph_correctness_passed(report)
    return report


def measure_graph_gap(session: Any, *, warmup: int = 5, timed: int = 20, repeats: int = 3) -> dict[str, Any]:
    """Repeated graph timing from the same prefilled state (the reference's
    ``measure_graph_gap``): per repeat, warm up, restore, time ``timed`` one-step
    replays; returns the per-token wall and device-event distributions, the
    host share and the kernels per step.  Leaves the session at its start state."""
    import torch  # noqa: PLC0415

    if session.graph is None:
        session.capture()
    warmup, timed = max(int(warmup), MIN_WARMUP), max(int(timed), MIN_TIMED)
    pos0, tok0 = _state(session)
    wall, event = [], []
    for _ in range(int(repeats)):
        session.set_position(pos0, tok0)
        session.replay(warmup, synchronize=False)
        torch.cuda.synchronize(session.device)
        session.set_position(pos0, tok0)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(session.device)
        e0.record()
        t0 = time.perf_counter()
        for _ in range(timed):
            session.replay(1, synchronize=False)
        e1.record()
        torch.cuda.synchronize(session.device)
        wall.append((time.perf_counter() - t0) * 1e3 / timed)
        event.append(e0.elapsed_time(e1) / timed)
    session.set_position(pos0, tok0)
    w, e = summarize(wall), summarize(event)
    host = max(w["p50"] - e["p50"], 0.0)
    return {
        "status": "measured",
        "method": "perf_counter wall + device events around timed one-step graph replays, per repeat",
        "wall_p50_ms": w["p50"], "wall_p99_ms": w["p99"],
        "gpu_p50_ms": e["p50"], "gpu_p99_ms": e["p99"],
        "gpu_busy_ms": e["p50"],
        "host_p50_ms": host,
        "host_share_pct": round(100.0 * host / w["p50"], 1) if w["p50"] else None,
        "kernels_per_call": session.launches_per_step,
        "stats": {"wall": w, "gpu_event": e},
        "warmup": warmup, "timed": timed, "repeats": int(repeats),
    }
