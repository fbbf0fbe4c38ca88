"""Shared test helpers (tolerances, comparisons, seeded inputs)."""

from __future__ import annotations

import torch

# The north-star tolerance for fp16 GEMV and attention outputs (rtol 2e-2, atol 2e-3).
RTOL = 2e-2
ATOL = 2e-3
# The reference's frozen kernel gate (src/lemoq/kernels/moe_grouped.py:64-72).
GATE_ATOL = 1e-3
GATE_RTOL = 1e-3
GATE_SLACK = 1.5


def max_abs(a, b) -> float:
    return float((a.double().cpu() - b.double().cpu()).abs().max())


def assert_close(got, ref, *, rtol: float = RTOL, atol: float = ATOL, what: str = "") -> None:
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    assert g.shape == r.shape, (what, tuple(g.shape), tuple(r.shape))
    assert torch.isfinite(g).all(), what + ": non-finite output"
    ok = torch.allclose(g, r, rtol=rtol, atol=atol)
    assert ok, "%s: max |diff| %.3e (rtol %g, atol %g)" % (what, float((g - r).abs().max()), rtol, atol)


def assert_gate(got, oracle64, baseline, *, what: str = "") -> None:
    """Reference K1 gate: err(kernel) <= 1.5 * err(baseline) (both vs fp64), plus allclose."""
    e_k = max_abs(got, oracle64)
    e_b = max_abs(baseline, oracle64)
    assert e_k <= GATE_SLACK * e_b + 1e-6, "%s: kernel err %.3e > %.1f x baseline err %.3e" % (
        what, e_k, GATE_SLACK, e_b)
    assert_close(got, oracle64, rtol=GATE_RTOL, atol=GATE_ATOL, what=what)


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(*shape, seed: int, std: float = 1.0, dtype=torch.float32):
    return (torch.randn(shape, generator=gen(seed), dtype=torch.float32) * std).to(dtype)
