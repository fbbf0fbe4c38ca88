"""Shared test helpers (tolerances, comparisons, seeded inputs)."""

from __future__ import annotations

import numpy as np
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


def kv_rows_vs_oracle(what, gpu_kv, gpu_rows, ref_kv, ref_rows, T, *, rows_close=True):
    """The KV-INT8 bytes of one layer's T prompt rows against the oracle's prefill:
    (1) with ``rows_close``, the GPU's fp16 k / v rows (after k_norm and RoPE)
        against the oracle's: every element within 2e-2 of the row's largest
        magnitude (RoPE's x*cos + rotate(x)*sin can cancel to a small value
        while carrying the absolute rounding of its terms, so an elementwise
        relative bound would not apply): for layer 0, whose inputs are the same
        embedding rows on both sides
        (deeper layers inherit every earlier difference, a near-tied routing
        choice included, so their rows are compared through (2) and (3) only);
    (2) the GPU's codes and scales bit-exact against the oracle's quantisation of
        the GPU's own fp16 rows, on every row;
    (3) on every row whose fp16 input equals the oracle's bit for bit, codes and
        scales bit-exact against the oracle's cache; the other rows (inputs that
        differ by an fp16 ulp after a different fp32 summation order) are counted
        and printed."""
    from oracle import quant as oq  # noqa: PLC0415

    for name, idx in (("k", 0), ("v", 1)):
        g16 = gpu_rows[idx].cpu()  # (heads, T, D)
        r16 = ref_rows[idx]
        NH, _, D = g16.shape
        if rows_close:
            err = (g16.float() - r16.float()).abs().amax(-1)
            scale = r16.float().abs().amax(-1)
            worst = float((err / scale.clamp_min(1e-6)).max())
            assert bool((err <= 2e-2 * scale).all()), "%s %s rows: worst error %.3e of the row scale" % (
                what, name, worst)
        gc, gs = gpu_kv[name + "c"][:, :T].cpu(), gpu_kv[name + "s"][:, :T].cpu()
        qc, qs = oq.kv_quantize_rows(g16.reshape(-1, D).numpy())
        assert np.array_equal(gc.reshape(-1, D).numpy(), qc), (what, name, "codes vs own rows")
        assert np.array_equal(gs.reshape(-1).numpy().view(np.uint16), qs.view(np.uint16)), (what, name)
        same = (g16.view(torch.int16) == r16.view(torch.int16)).all(-1)  # (heads, T)
        rc, rs = ref_kv[name + "c"][:, :T], ref_kv[name + "s"][:, :T]
        assert torch.equal(gc[same], rc[same]), (what, name, "codes on rows with identical input")
        assert torch.equal(gs[same].view(torch.int16), rs[same].view(torch.int16)), (what, name)
        n_same = int(same.sum())
        print("%s %s: %d of %d rows with the oracle's fp16 input, bytes bit-exact there; %d excused"
              % (what, name, n_same, NH * T, NH * T - n_same))
