#!/usr/bin/env python3
"""Decode-step benchmark of the lemoq MI355X build (one GPU).

Workload: the OLMoE-1B-7B-shaped batch-1 decode step of the reference's
canonical cell (w8a16 g128 attention + experts, W8 lm_head, KV-INT8 cache,
split-KV attention, one graph per step): seeded random weights, prompt of
``ctx`` copies of token id 1, then greedy decode steps replayed from one
captured hipGraph.  The reference quotes this as ms/token at ctx 1024 and 4096
(README_EN.md:66-71 of LeanMoE-Quant, RTX 5090).

Printed: ONE JSON line on stdout.  ``value`` is ms/token at ``--ctx``: the p50
of ``--steps`` per-step times (an event between consecutive replays, after
``--warmup`` replays), the reference's timing convention; ``ms_per_step_mean``
is the wall clock over exactly ``--steps`` back-to-back replays, synchronised on
both sides; ``ms_per_token_graph8`` is the p50 over launches of graphs that
hold 8 decode steps each, divided by 8 (not the headline: the reference
replays one step per graph).  The line also carries the second context, the step's HBM roofline
fraction, per-kernel cold timings, the dominant kernel's roofline
(``roofline``), the CPU path on this host (``cpu_baseline``: the oracle's
ms/token p50/p99 on all threads and on one, at both contexts, and the C1-C4
operators' microseconds beside the GPU's) and, per context, the batched
prefill's TTFT with E2E-32/128 beside the reference's published values
(``prefill``).  Progress goes to stderr.

``--mode kernels`` runs only the weights + isolated kernel timings.
``--mode traffic`` is the short form profiled under ``rocprofv3 --pmc``: a
copy of known size (the counter calibration), then the isolated kernels over
a synthetic KV cache at ``--ctx`` (no prefill); it prints the dispatch plan.
``--summarize-pmc FETCH_CSV WRITE_CSV PLAN_JSON`` (CPU only) turns the two
counter passes into per-kernel HBM bytes per launch: profiles/traffic.json,
which fills ``roofline.traffic``, and a markdown table beside it.
``--summarize-trace TRACE_CSV`` (CPU only) splits a ``rocprofv3
--kernel-trace`` of a full run per kernel into the graph's launches and the
kernel table's cold isolated launches (the latter are what ``roofline`` and
``kernels`` time).  ``--mode step`` prefills ``--ctx`` once and replays the step ``--warmup`` +
``--steps`` times (nothing else: the form profiled for the in-graph kernel
times).  ``--mode prefill`` times only the batched prefill (TTFT) at ``--ctx`` (and
``--ctx2``); ``--summarize-prefill TRACE_CSV --ctx T`` (CPU only) turns a
``rocprofv3 --kernel-trace`` of it into a per-kernel table with each kernel's
FLOP rate against the MI355X dense fp16 matrix peak.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "leanmoe-quant_amd")
for _p in (REPO, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "ms/token decode step, OLMoE-shape w8a16+KV-INT8 @ctx1024/4096; % HBM roofline"
HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X published dense fp16 matrix peak
REFERENCE_RTX5090_MS = {"1024": 1.4602, "4096": 1.6075}  # README_EN.md:71 (not this hardware)
# Canonical-cell TTFT p50 and E2E-32 of the reference (RESULTS.md:136-141, RTX 5090, not this hardware).
REFERENCE_RTX5090_TTFT_MS = {"1024": 84.4366, "4096": 158.3072}
REFERENCE_RTX5090_E2E32_MS = {"1024": 131.16, "4096": 209.75}
KV_BYTES_PER_TOKEN_LAYER = 16 * (128 + 2) * 2  # 16 heads x (128 codes + fp16 scale) x (K, V)
KV_F16_BYTES_PER_TOKEN_LAYER = 16 * 128 * 2 * 2  # 16 heads x 128 fp16 values x (K, V)
# the reference's cell with KV-INT8 off (EXP-p5-01-kv-int8.md:140-143; RTX 5090, not this hardware)
REFERENCE_RTX5090_KV_F16_MS = {"1024": 1.4689, "4096": 1.71798}


def log(msg: str) -> None:
    sys.stderr.write("[bench %7.1fs] %s\n" % (time.time() - _T0, msg))
    sys.stderr.flush()


_T0 = time.time()


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ctx", type=int, default=1024)
    ap.add_argument("--ctx2", type=int, default=4096, help="second context (0: skip)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--kernel-reps", type=int, default=4)
    ap.add_argument("--cpu-check-steps", type=int, default=32,
                    help="GPU steps checked against the CPU oracle (also its first timed steps)")
    ap.add_argument("--cpu-warmup", type=int, default=5, help="untimed CPU oracle steps / op calls")
    ap.add_argument("--cpu-timed", type=int, default=20, help="timed CPU oracle steps / op calls (all threads)")
    ap.add_argument("--cpu-timed-1t", type=int, default=20, help="timed CPU oracle steps on one thread")
    ap.add_argument("--no-cpu-ops", action="store_true", help="skip the per-operator CPU timings (C1-C4)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-formats", action="store_true", help="skip the weight-format GEMV timings")
    ap.add_argument("--no-kv-fp16", action="store_true", help="skip the fp16-cache (KV-INT8 off) step timing")
    ap.add_argument("--kv-cache", choices=("int8", "fp16"), default="int8",
                    help="--mode step: the decode cache kind (fp16 = the cell with KV-INT8 off)")
    ap.add_argument("--weights", choices=("w8a16", "w4a16"), default="w8a16",
                    help="--mode step: the cell's weights (w4a16: 4-bit attention and experts, fp16 lm_head)")
    ap.add_argument("--no-w4a16", action="store_true", help="skip the w4a16-cell step timing")
    ap.add_argument("--summarize-last", type=int, default=0,
                    help="--summarize-step: keep only the last N whole steps (0: all)")
    ap.add_argument("--mode", choices=("full", "kernels", "traffic", "prefill", "step"), default="full")
    ap.add_argument("--summarize-pmc", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "PLAN_JSON"))
    ap.add_argument("--summarize-prefill", metavar="KERNEL_TRACE_CSV",
                    help="per-kernel table of the prefills in a rocprofv3 kernel trace of --mode prefill at --ctx")
    ap.add_argument("--summarize-step", metavar="KERNEL_TRACE_CSV",
                    help="per-kernel table and timeline of the decode step in a rocprofv3 kernel trace of --mode step")
    ap.add_argument("--summarize-trace", metavar="KERNEL_TRACE_CSV",
                    help="per-kernel table of a rocprofv3 kernel trace of a full bench run: in-graph launches "
                         "and the cold isolated launches of the kernel table, separately")
    ap.add_argument("--profiles-dir", default=os.path.join(REPO, "profiles"))
    return ap.parse_args(argv)


# ---------------------------------------------------------------------------
# timing helpers
# ---------------------------------------------------------------------------
class Flusher:
    """Reads a buffer larger than the 256 MB Infinity Cache + L2 (evicts them) and
    measures the read bandwidth of that stream (the roofline denominator)."""

    def __init__(self, torch, hip, dev, nbytes: int = 1 << 30):
        self.torch, self.hip = torch, hip
        self.buf = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
        self.buf.fill_(1)
        self.nbytes = nbytes
        self.blocks = max(1, min(65536, nbytes // 16384))  # 16 KB shares: one 4 KB chunk per wave
        self.out = torch.empty((self.blocks,), dtype=torch.int32, device=dev)

    def flush(self) -> None:
        self.hip.call("lemoq_read_probe", self.hip.ptr(self.buf), self.nbytes, self.hip.ptr(self.out),
                      self.blocks, self.hip.stream_of())

    def read_bandwidth_gbs(self, reps: int = 10) -> float:
        torch = self.torch
        self.flush()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for a, b in evs:
            a.record()
            self.flush()
            b.record()
        torch.cuda.synchronize()
        ms = sorted(a.elapsed_time(b) for a, b in evs)
        return self.nbytes / (ms[len(ms) // 2] * 1e-3) / 1e9


def time_cold(torch, flusher, launches, reps: int) -> dict:
    """Per-launch duration of back-to-back launches: flush the caches, then time
    one pass over ``launches`` (callables enqueueing one kernel each on the
    current stream, one per layer so every launch reads cold weights) between
    two events; ``reps`` passes.  No event sits between the kernels, so the
    average is comparable with the profiler's per-kernel duration."""
    evs = []
    for _ in range(reps):
        flusher.flush()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for fn in launches:
            fn()
        b.record()
        evs.append((a, b))
    torch.cuda.synchronize()
    us = sorted(a.elapsed_time(b) * 1e3 / len(launches) for a, b in evs)
    return {"avg_us": sum(us) / len(us), "p50_us": us[len(us) // 2], "min_us": us[0],
            "launches": reps * len(launches)}


# ---------------------------------------------------------------------------
# isolated kernels of the step (the same entry points the step executor calls)
# ---------------------------------------------------------------------------
READ_FLOOR = "read floor (gate/up bytes, read only)"


def kernel_table(torch, hip, w, sess, flusher, reps: int, floors: bool = True) -> dict:
    s = w.shape
    H, HD, D, F, E, K, g = s.hidden, s.heads * s.head_dim, s.head_dim, s.ffn, s.num_experts, s.top_k, s.group_size
    P, st = hip.ptr, hip.stream_of
    L = w.layers
    nl = len(L)
    filled = int(sess.filled.item())
    S = sess.max_seq
    w8 = lambda rows, cols: rows * cols + rows * (cols // g) * 2  # noqa: E731
    dev = sess.device
    scratch = {
        "h": torch.randn((H,), device=dev).to(torch.float16),
        "y": torch.empty((max(s.vocab, 3 * HD),), dtype=torch.float16, device=dev),
        "ids": sess.top_i.clone(),
        "tw": sess.top_w.clone(),
        "act": sess.act.clone(),
        "xn": torch.empty((H,), dtype=torch.float16, device=dev),
        "h2": torch.empty((H,), dtype=torch.float16, device=dev),
        "lg": torch.empty((E,), dtype=torch.float16, device=dev),
        "tok": torch.zeros((1,), dtype=torch.int64, device=dev),
        "pos": torch.zeros((1,), dtype=torch.int64, device=dev),
        "fill": torch.zeros((1,), dtype=torch.int32, device=dev),
        "ids2": sess.top_i.clone(),
        "tw2": sess.top_w.clone(),
        "act2": sess.act.clone(),
        "fixed_ids": torch.arange(K, dtype=torch.int64, device=dev) * (E // K),
        "probe": torch.empty((1024,), dtype=torch.int32, device=dev),
    }
    kv = sess.kv
    qk_scale = (1.0 / math.sqrt(D)) * 1.4426950408889634
    specs = {}

    def add(name, nbytes, launches, kernels):
        specs[name] = (nbytes, launches, kernels)

    add("moe_gate_up_w8_routed", K * w8(2 * F, H) + H * 2 + E * 2 + K * F * 2,
        [lambda i=i: hip.call("lemoq_moe_gate_up_w8_routed", P(scratch["h"]), P(L[i].gu_codes), P(L[i].gu_scale),
                               P(sess.router_logits), K, int(s.norm_topk_prob), E, F, H, g, P(scratch["act"]),
                               P(scratch["ids"]), P(scratch["tw"]), st()) for i in range(nl)],
        ["moe_gate_up_kernel"])
    if floors:
        # The same launch given the ids (no routing before the weight loads), and a launch that only
        # reads the same number of bytes: the single-launch read floor the routed kernel is held to.
        # (Left out of the traffic pass, whose cache flushes are read_probe dispatches too.)
        add("moe_gate_up_w8 (ids given)", K * w8(2 * F, H) + H * 2 + K * 8 + K * F * 2,
            [lambda i=i: hip.call("lemoq_moe_gate_up_w8", P(scratch["h"]), P(L[i].gu_codes), P(L[i].gu_scale),
                                   P(scratch["fixed_ids"]), K, E, F, H, g, P(scratch["act2"]), st())
             for i in range(nl)],
            ["moe_gate_up_kernel"])
        gu_bytes = (K * w8(2 * F, H) + H * 2 + E * 2 + K * F * 2) // 16 * 16
        add(READ_FLOOR, gu_bytes,
            [lambda i=i: hip.call("lemoq_read_probe", P(L[i].gu_codes), gu_bytes, P(scratch["probe"]), 1024, st())
             for i in range(nl)],
            ["read_probe_kernel"])
        # the same floor at the down and qkv launches' byte counts (each layer's gate/up codes
        # serve as 16 distinct source buffers)
        for label, nb in (("down", K * w8(H, F) + K * F * 2 + 3 * H * 2), ("qkv", w8(3 * HD, H) + 2 * H * 2 + 3 * HD * 2)):
            nb16 = nb // 16 * 16
            add("read floor (%s bytes, read only)" % label, nb16,
                [lambda i=i, nb16=nb16: hip.call("lemoq_read_probe", P(L[i].gu_codes), nb16, P(scratch["probe"]),
                                                 1024, st()) for i in range(nl)],
                ["read_probe_kernel"])
    add("moe_down_w8", K * w8(H, F) + K * F * 2 + 3 * H * 2,
        [lambda i=i: hip.call("lemoq_moe_down_w8", P(scratch["act"]), P(L[i].dn_codes), P(L[i].dn_scale),
                               P(scratch["ids"]), P(scratch["tw"]), K, E, H, F, g, P(scratch["h"]),
                               P(scratch["y"]), st()) for i in range(nl)],
        ["moe_down_kernel"])
    add("gemv_w8 qkv (+input RMSNorm)", w8(3 * HD, H) + 2 * H * 2 + 3 * HD * 2,
        [lambda i=i: hip.call("lemoq_gemv_w8_fused", P(scratch["h"]), None, 0, P(L[i].ln_in), s.eps, None,
                               P(L[i].qkv_codes), P(L[i].qkv_scale), 3 * HD, H, g, None, P(scratch["y"]), st())
         for i in range(nl)],
        ["gemv_w8_kernel"])
    ns = sess.num_splits
    add("attn_split_fused_i8 (filled=%d)" % filled,
        KV_BYTES_PER_TOKEN_LAYER * filled + 3 * HD * 2 + 2 * HD * 2 + 2 * D * 2 + s.heads * ns * (D + 2) * 4,
        [lambda i=i: hip.call("lemoq_attn_split_fused_i8", P(sess.qkv), s.heads, D, P(L[i].q_norm),
                               P(L[i].k_norm), s.eps, P(sess.cos_tab), P(sess.sin_tab), P(sess.pos),
                               P(kv[i]["kc"]), P(kv[i]["ks"]), P(kv[i]["vc"]), P(kv[i]["vs"]), S * D, S, ns,
                               qk_scale, P(sess.part_m), P(sess.part_l), P(sess.part_acc),
                               math.inf if s.clip_qkv is None else s.clip_qkv,
                               st())
         for i in range(nl)],
        ["attn_split_fused_i8_kernel"])
    # the same attention launch over the fp16 cache (KV-INT8 off): 16 layers' worth of fp16 rows
    # with the same filled length, random values
    kv16 = [(torch.randn((s.heads, S, D), device=dev).to(torch.float16),
             torch.randn((s.heads, S, D), device=dev).to(torch.float16)) for _ in range(nl)]
    add("attn_split_fused_f16 (filled=%d)" % filled,
        KV_F16_BYTES_PER_TOKEN_LAYER * filled + 3 * HD * 2 + 2 * HD * 2 + 2 * D * 2 + s.heads * ns * (D + 2) * 4,
        [lambda i=i: hip.call("lemoq_attn_split_fused_f16", P(sess.qkv), s.heads, D, P(L[i].q_norm),
                               P(L[i].k_norm), s.eps, P(sess.cos_tab), P(sess.sin_tab), P(sess.pos),
                               P(kv16[i][0]), P(kv16[i][1]), S * D, S, ns, qk_scale, P(sess.part_m),
                               P(sess.part_l), P(sess.part_acc), math.inf if s.clip_qkv is None else s.clip_qkv,
                               st())
         for i in range(nl)],
        ["attn_split_fused_f16_kernel"])
    if sess.attn_output_fused:
        npart = HD // 512
        add("attn_merge_o_proj_w8", w8(H, HD) + s.heads * ns * (D + 2) * 4 + npart * H * 4,
            [lambda i=i: hip.call("lemoq_attn_merge_o_proj_w8", P(sess.part_m), P(sess.part_l), P(sess.part_acc),
                                   s.heads, ns, D, P(L[i].o_codes), P(L[i].o_scale), H, g, P(sess.o_part), st())
             for i in range(nl)],
            ["merge_oproj_kernel"])
        add("router_logits_resid", E * H * 2 + npart * H * 4 + 4 * H * 2 + E * 2,
            [lambda i=i: hip.call("lemoq_router_logits_resid", P(sess.o_part), npart, P(scratch["h"]),
                                   P(L[i].ln_post), s.eps, H, P(L[i].router), E, P(scratch["h2"]), P(scratch["xn"]),
                                   P(scratch["lg"]), st()) for i in range(nl)],
            ["router_resid_kernel"])
    else:
        add("attn_merge", s.heads * ns * (D + 2) * 4 + HD * 2,
            [lambda: hip.call("lemoq_attn_merge", P(sess.part_m), P(sess.part_l), P(sess.part_acc), s.heads, ns, D,
                              P(sess.attn), st())] * nl,
            ["attn_merge_kernel"])
        add("gemv_w8 o_proj (+residual)", w8(H, HD) + HD * 2 + 2 * H * 2,
            [lambda i=i: hip.call("lemoq_gemv_w8_fused", P(sess.attn), None, 0, None, s.eps, None,
                                   P(L[i].o_codes), P(L[i].o_scale), H, HD, g, P(scratch["h"]), P(scratch["y"]),
                                   st())
             for i in range(nl)],
            ["gemv_w8_kernel"])
        add("router_logits", E * H * 2 + 3 * H * 2 + E * 2,
            [lambda i=i: hip.call("lemoq_router_logits", P(scratch["h"]), P(L[i].ln_post), s.eps, H, P(L[i].router),
                                   E, P(scratch["xn"]), P(scratch["lg"]), st()) for i in range(nl)],
            ["router_logits_kernel"])
    add("gemv_w8 lm_head + argmax (2 launches)", w8(s.vocab, H) + 2 * H * 2 + s.vocab * 2,
        [lambda: hip.call("lemoq_lm_head_argmax_w8", P(scratch["h"]), P(w.final_norm), s.eps, P(w.lm_codes),
                          P(w.lm_scale), s.vocab, H, g, P(scratch["y"]), P(sess.am_val), P(sess.am_idx),
                          int(sess.am_val.numel()), P(scratch["tok"]), P(scratch["pos"]), P(scratch["fill"]),
                          None, 0, None, 0, st())],
        ["gemv_w8_kernel", "argmax_advance_kernel"])
    out = {}
    for name, (nbytes, launches, kernels) in specs.items():
        r = time_cold(torch, flusher, launches, reps)
        r["bytes"] = int(nbytes)
        r["dispatch_kernels"] = kernels
        r["gbs"] = nbytes / (r["avg_us"] * 1e-6) / 1e9
        r["frac_of_peak"] = r["gbs"] / HBM_PEAK_GBS
        out[name] = r
        log("kernel %-36s %8.2f us avg  %7.1f GB/s" % (name, r["avg_us"], r["gbs"]))
    return out


# ---------------------------------------------------------------------------
# decode timing
# ---------------------------------------------------------------------------
def measure_prefill(torch, sess, warmup: int = 2, timed: int = 7) -> dict:
    """TTFT as the reference measures it (``_measure_static_prefill``,
    ``benchmarks/runner.py:1045-1064``): wall time of a whole prefill (cache
    reset, the batched forward of the prompt, greedy pick of the seed token)
    between device synchronisations; ``warmup`` untimed, p50 of ``timed``.
    Leaves the session prefilled."""
    for _ in range(warmup):
        sess.prefill()
    torch.cuda.synchronize()
    samples = []
    for _ in range(timed):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        sess.prefill()
        torch.cuda.synchronize()
        samples.append((time.perf_counter() - t0) * 1e3)
    samples.sort()
    return {"p50": samples[len(samples) // 2], "min": samples[0], "max": samples[-1], "runs": timed}


MULTI_STEPS = 8  # decode steps per graph of the multi-step measurement


def measure_repeats(torch, sess, *, warmup: int, timed: int, repeats: int) -> dict:
    """The reference's repeated graph timing (``measure_graph_gap``,
    ``benchmarks/cudagraph.py:420-495``), run by ``lemoq.model.graph_session``:
    each repeat starts from the same prefilled state (position and seed token
    restored, outside the timed window), replays ``warmup`` steps untimed,
    restores the state again, then times ``timed`` replays with host wall time
    and device events; returns the per-repeat ms/token of both and their spread
    ((max - min) / min).  The KV slots past the prompt are rewritten by each
    repeat's own steps, so every repeat decodes the same positions from the
    same cache."""
    from lemoq.model.graph_session import measure_graph_gap  # noqa: PLC0415

    gap = measure_graph_gap(sess, warmup=warmup, timed=timed, repeats=repeats)
    wall, event = gap["stats"]["wall"]["samples"], gap["stats"]["gpu_event"]["samples"]
    return {"warmup": gap["warmup"], "timed": gap["timed"], "wall_ms": wall, "event_ms": event,
            "wall_spread": (max(wall) - min(wall)) / min(wall),
            "event_spread": (max(event) - min(event)) / min(event),
            "host_share_pct": gap["host_share_pct"], "method": gap["method"]}


def time_decode(torch, w, ctx: int, steps: int, warmup: int, extra: int):
    from lemoq.model.olmoe import DecodeSession

    groups = max(8, steps // MULTI_STEPS)
    sess = DecodeSession(w, [1] * ctx, max_new_tokens=warmup + 2 * steps + groups * MULTI_STEPS + extra + 4,
                         kv_cache="int8")
    sess.capture()
    ttft = measure_prefill(torch, sess)
    log("ctx %d: batched prefill (TTFT) p50 %.3f ms over %d runs" % (ctx, ttft["p50"], ttft["runs"]))
    # TTFT on a seeded random prompt too: tokens route to all 64 experts, so the
    # prefill streams every expert's weights (with ctx ones all rows pick the same 8)
    rnd = DecodeSession(w, torch.randint(0, w.shape.vocab, (ctx,), generator=torch.Generator().manual_seed(ctx)),
                        max_new_tokens=2, kv_cache="int8")
    rnd.capture()
    ttft_rnd = measure_prefill(torch, rnd)
    del rnd
    log("ctx %d: batched prefill of a random prompt (TTFT) p50 %.3f ms" % (ctx, ttft_rnd["p50"]))
    # the reference's per-cell gate (benchmarks/cudagraph.py:298-339): eager steps against graph
    # replays from the prefilled state, KL <= 1e-5 and identical tokens; state restored after
    from lemoq.model.graph_session import graph_correctness  # noqa: PLC0415

    gate = graph_correctness(sess, steps=8)
    log("ctx %d: graph == eager gate %s (KL %.1e, bitwise %s)" % (ctx, "PASS" if gate["passed"] else "FAIL",
                                                                   gate["kl"], gate["bitwise"]))
    repeats = measure_repeats(torch, sess, warmup=max(warmup, 5), timed=max(steps, 20), repeats=3)
    log("ctx %d: %d repeats x %d replays from the prefilled state: event ms/token %s (spread %.2f%%)"
        % (ctx, len(repeats["event_ms"]), repeats["timed"], ", ".join("%.4f" % v for v in repeats["event_ms"]),
           100.0 * repeats["event_spread"]))
    sess.replay(warmup)
    filled0 = int(sess.filled.item())
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        sess.replay(1, synchronize=False)
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    dev_ms = e0.elapsed_time(e1)
    # Per-step latency distribution: a second pass with an event between replays.
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    evs[0].record()
    for i in range(steps):
        sess.replay(1, synchronize=False)
        evs[i + 1].record()
    torch.cuda.synchronize()
    per = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(steps))
    p50, p99 = per[len(per) // 2], per[min(len(per) - 1, int(round(0.99 * (len(per) - 1))))]
    # Multi-step graphs: MULTI_STEPS decode steps per graph launch, an event
    # between launches (not the headline: the reference replays one step per graph).
    sess.capture(steps_per_graph=MULTI_STEPS)
    gev = [torch.cuda.Event(enable_timing=True) for _ in range(groups + 1)]
    gev[0].record()
    for i in range(groups):
        sess.replay(MULTI_STEPS, synchronize=False)
        gev[i + 1].record()
    torch.cuda.synchronize()
    per_group = sorted(gev[i].elapsed_time(gev[i + 1]) / MULTI_STEPS for i in range(groups))
    filled_avg = filled0 + (steps - 1) / 2.0
    step_bytes = w.shape.weight_bytes_per_token() + KV_BYTES_PER_TOKEN_LAYER * w.shape.layers * filled_avg
    res = {
        "ctx": ctx,
        "ms_per_token": wall_ms / steps,
        "device_ms_per_token": dev_ms / steps,
        "tokens_per_s": steps / (wall_ms * 1e-3),
        "host_share": max(0.0, (wall_ms - dev_ms) / wall_ms),
        "filled_first": filled0,
        "step_bytes": int(step_bytes),
        "launches_per_step": sess.launches_per_step,
        "step_ms_p50": p50,
        "step_ms_p99": p99,
        "ms_per_token_graph%d" % MULTI_STEPS: per_group[len(per_group) // 2],
        "ttft": ttft,
        "ttft_random_prompt": ttft_rnd,
        "repeats": repeats,
        "graph_gate": {k: gate[k] for k in ("kl", "top1_agreement", "seed_token_match", "token_sequence_match",
                                            "bitwise", "passed", "steps")},
        # the reference's per-token figure: p50 over the repeats of the wall-clock
        # mean per replay (runner.py:984, gap["stats"]["wall"]["p50"])
        "ms_per_token_repeats_p50": sorted(repeats["wall_ms"])[len(repeats["wall_ms"]) // 2],
    }
    log("ctx %d: %.4f ms/token wall, %.4f device, %d steps; per-step p50 %.4f p99 %.4f ms; "
        "%d-step graphs p50 %.4f ms/token over %d launches"
        % (ctx, res["ms_per_token"], res["device_ms_per_token"], steps, p50, p99, MULTI_STEPS,
           res["ms_per_token_graph%d" % MULTI_STEPS], groups))
    return sess, res


def time_kv_fp16(torch, w, ctx: int, steps: int, warmup: int, read_bw: float) -> dict:
    """The step over the fp16 cache (the reference's cell with KV-INT8 off): the
    same repeated timing as the headline (3 repeats x ``steps`` replays from the
    prefilled state of ``[1] * ctx``), and its bytes with fp16 KV rows."""
    from lemoq.model.olmoe import DecodeSession

    sess = DecodeSession(w, [1] * ctx, max_new_tokens=max(warmup, 5) + max(steps, 20) + 4, kv_cache="fp16")
    sess.capture()
    sess.prefill()
    rep = measure_repeats(torch, sess, warmup=max(warmup, 5), timed=max(steps, 20), repeats=3)
    ms = sorted(rep["wall_ms"])[1]
    dev_ms = sorted(rep["event_ms"])[1]
    filled_avg = ctx + 1 + (rep["timed"] - 1) / 2.0
    nbytes = w.shape.weight_bytes_per_token() + KV_F16_BYTES_PER_TOKEN_LAYER * w.shape.layers * filled_avg
    launches = sess.launches_per_step
    del sess
    res = {"ms_per_token_repeats_p50": ms, "device_ms_per_token": dev_ms, "wall_spread": rep["wall_spread"],
           "step_bytes": int(nbytes), "step_hbm_frac_of_measured": nbytes / (dev_ms * 1e-3) / 1e9 / read_bw,
           "launches_per_step": launches}
    log("ctx %d fp16 cache: %.4f ms/token (repeats p50), device %.4f" % (ctx, ms, dev_ms))
    return res


def time_w4a16(torch, shape, seed: int, dev, ctx: int, steps: int, warmup: int, read_bw: float) -> dict:
    """The reference's w4a16 cell (4-bit attention and experts, router and lm_head
    fp16, KV-INT8; ``--bit-width w4a16``, benchmarks/runner.py:393-412,451-482) on
    the same shape: the prompt ``[1] * ctx`` fed through the step (the batched
    prefill runs W8 weights), then the headline's repeated timing, and the
    cell's bytes per step (``lemoq.bytes`` at 4 bits)."""
    from lemoq.bytes import step_bytes
    from lemoq.model.olmoe import DecodeSession, OlmoeW8Weights

    w4 = OlmoeW8Weights.random(shape, seed=seed, device=dev, bits=4, lm_head="fp16")
    sess = DecodeSession(w4, [1] * ctx, max_new_tokens=max(warmup, 5) + max(steps, 20) + 4, kv_cache="int8")
    sess.capture()
    ttft = measure_prefill(torch, sess)  # batched prefill of the ctx-ones prompt; leaves the session prefilled
    rep = measure_repeats(torch, sess, warmup=max(warmup, 5), timed=max(steps, 20), repeats=3)
    ms = sorted(rep["wall_ms"])[1]
    dev_ms = sorted(rep["event_ms"])[1]
    filled_avg = ctx + 1 + (rep["timed"] - 1) / 2.0
    nbytes = step_bytes(shape, 0, bits=w4.weight_bits()) + KV_BYTES_PER_TOKEN_LAYER * shape.layers * filled_avg
    launches = sess.launches_per_step
    del sess, w4
    torch.cuda.empty_cache()
    res = {"ms_per_token_repeats_p50": ms, "device_ms_per_token": dev_ms, "wall_spread": rep["wall_spread"],
           "step_bytes": int(nbytes), "step_hbm_frac_of_measured": nbytes / (dev_ms * 1e-3) / 1e9 / read_bw,
           "launches_per_step": launches, "ttft_ms_p50": ttft["p50"]}
    log("ctx %d w4a16: %.4f ms/token (repeats p50), device %.4f, TTFT %.3f ms" % (ctx, ms, dev_ms,
                                                                               ttft["p50"]))
    return res


def _p50_p99(samples: list) -> tuple:
    s = sorted(samples)
    return s[len(s) // 2], s[min(len(s) - 1, int(round(0.99 * (len(s) - 1))))]


def _pad_kv(torch, kv: list, slots: int) -> list:
    """Host KV-INT8 snapshot widened to ``slots`` cache slots (the CPU oracle keeps
    stepping past the GPU session's capacity); new slots hold code 0, scale 1."""
    out = []
    for layer in kv:
        d = {}
        for name, t in layer.items():
            S = int(t.shape[1])
            if S >= slots:
                d[name] = t
                continue
            shape = list(t.shape)
            shape[1] = slots
            fill = 1.0 if name in ("ks", "vs") else 0
            big = torch.full(shape, fill, dtype=t.dtype)
            big[:, :S] = t
            d[name] = big
        out.append(d)
    return out


def _oracle_steps(od, first_token: int, pos: int, n: int, forced: list) -> tuple:
    """n oracle decode steps from (first_token, pos); step i consumes forced[i] when
    given, else the oracle's own greedy token.  Returns (ms per step, logits)."""
    times, logits, tok = [], [], int(first_token)
    for i in range(n):
        if i < len(forced):
            tok = int(forced[i])
        t = time.perf_counter()
        lg = od.step(tok, pos + i)
        times.append(1e3 * (time.perf_counter() - t))
        logits.append(lg)
        tok = od.greedy(lg)
    return times, logits


def cpu_baseline(torch, host, snap, gpu_tokens, gpu_logits, *, warmup: int, timed: int, timed_1t: int,
                 snap2=None) -> dict:
    """The CPU path (the torch-CPU oracle restating the reference's ``backend="oracle"``
    operators and the HF glue) on this host's cores: the full decode step from the GPU's
    KV snapshot, teacher-forced on the GPU's greedy tokens (the parity check of every
    bench run), ``warmup`` untimed + ``timed`` timed steps, p50 / p99 per step
    (``benchmarks/timing.py:19-69`` of the reference), on all threads and on one."""
    from oracle.olmoe import OracleDecoder

    kv, token, pos = snap
    n_all = warmup + timed
    slots = pos + max(n_all, len(gpu_logits)) + warmup + timed_1t + 2
    if snap2 is not None:
        slots = max(slots, snap2[2] + n_all + 2)
    t = time.time()
    od = OracleDecoder(host, slots, kv=_pad_kv(torch, kv, slots))
    threads = torch.get_num_threads()
    log("cpu oracle ready in %.1fs (%d threads)" % (time.time() - t, threads))
    seq = [token] + list(gpu_tokens)
    n = max(n_all, len(gpu_logits))
    times, logits = _oracle_steps(od, token, pos, n, seq)
    agree, flips, max_kl, max_diff = 0, [], 0.0, 0.0
    for i, got in enumerate(gpu_logits):
        ref, g = logits[i].double(), got.double()
        p, q = torch.log_softmax(ref, -1), torch.log_softmax(g, -1)
        kl = float((p.exp() * (p - q)).sum())
        diff = float((ref - g).abs().max())
        top = torch.topk(ref, 2).values
        if int(torch.argmax(ref)) == int(torch.argmax(g)):
            agree += 1
        else:
            flips.append({"step": i, "margin": float(top[0] - top[1]), "logit_diff": diff})
        max_kl, max_diff = max(max_kl, kl), max(max_diff, diff)
    t_all = times[warmup:]
    p50, p99 = _p50_p99(t_all)
    log("cpu oracle ctx %d: p50 %.1f p99 %.1f ms/token on %d threads (%d timed after %d warmup)"
        % (pos, p50, p99, threads, len(t_all), warmup))
    # one thread: the same oracle keeps decoding (its own greedy tokens) from where it stopped
    torch.set_num_threads(1)
    try:
        t1, _ = _oracle_steps(od, od.greedy(logits[-1]), pos + n, warmup + timed_1t, [])
    finally:
        torch.set_num_threads(threads)
    p50_1t, p99_1t = _p50_p99(t1[warmup:])
    log("cpu oracle: p50 %.1f p99 %.1f ms/token on 1 thread (%d timed after %d warmup)"
        % (p50_1t, p99_1t, timed_1t, warmup))
    res = {
        "value": p50,
        "unit": "ms/token",
        "cores": int(threads),
        "stat": "p50",
        "p99": p99,
        "mean": sum(t_all) / len(t_all),
        "warmup": warmup,
        "timed": len(t_all),
        "value_1thread": p50_1t,
        "p99_1thread": p99_1t,
        "timed_1thread": timed_1t,
        "cpu_model": _cpu_model(),
        "kind": "port",
        "sample": "%d decode steps (%d warmup) of the full OLMoE-1B-7B-shaped w8a16+KV-INT8 model by the "
                  "torch-CPU oracle from the GPU's KV snapshot at position %d, fed the GPU's greedy tokens; "
                  "then %d steps (%d warmup) on one thread" % (n, warmup, pos, warmup + timed_1t, warmup),
        "host_cpu_count": os.cpu_count(),
        "parity": {"steps": len(gpu_logits), "argmax_agree": agree, "flips": flips, "max_kl": max_kl,
                   "max_logit_diff": max_diff},
    }
    if snap2 is not None:
        kv2, token2, pos2 = snap2
        od.kv = _pad_kv(torch, kv2, slots)
        t2, _ = _oracle_steps(od, token2, pos2, n_all, [])
        a, b = _p50_p99(t2[warmup:])
        res["ctx2"] = {"position": pos2, "p50": a, "p99": b, "timed": timed, "warmup": warmup}
        log("cpu oracle ctx %d: p50 %.1f p99 %.1f ms/token on %d threads" % (pos2, a, b, threads))
    return res


def cpu_ops_baseline(torch, host, *, warmup: int, timed: int, seed: int = 0) -> dict:
    """Benchmark configs C1-C4 as single operators of the reference's CPU path (the
    torch oracle backend, ``moe_grouped_quant.py:476-477,520-523``, ``attn_decode.py:581-586``,
    ``reference.py:50-60``; dense GEMVs dequantise the weight on every call as that
    oracle does), p50 / p99 microseconds per call on this host's threads.  C1 uses the
    model's layer-0 router and experts with norm_topk_prob=True; x ~ N(0, 1)."""
    from oracle import ops
    from oracle import quant as oq

    s = host.shape
    g = s.group_size
    L0 = host.layers[0]
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((1, s.hidden), generator=gen).to(torch.float16)
    gamma = (torch.rand((s.hidden,), generator=gen) + 0.5).to(torch.float16)
    D, NH = s.head_dim, s.heads
    HD = NH * D

    def timeit(fn) -> dict:
        ts = []
        for i in range(warmup + timed):
            t = time.perf_counter()
            fn()
            if i >= warmup:
                ts.append(1e6 * (time.perf_counter() - t))
        a, b = _p50_p99(ts)
        return {"cpu_us_p50": a, "cpu_us_p99": b}

    def c1():
        _, tw, ti = ops.route(x, L0.router, s.top_k, True)
        ops.grouped_moe_w8(x.reshape(-1), L0.gu_codes, L0.gu_scale, L0.dn_codes, L0.dn_scale, g,
                           ti.reshape(-1), tw.reshape(-1))

    out = {"C1 grouped MoE (router + top-8 of 64, w8 gate/up + down)": timeit(c1)}
    for ctx in (1024, 4096):
        q = torch.randn((NH, D), generator=gen).to(torch.float16)
        k = torch.randn((NH, ctx, D), generator=gen).to(torch.float16)
        v = torch.randn((NH, ctx, D), generator=gen).to(torch.float16)
        out["C2 split-KV fp16 attention ctx %d" % ctx] = timeit(
            lambda: ops.split_kv_oracle(q, k, v, ctx, num_splits=ctx // 256).to(torch.float16))
    for ctx in (4096, 16384):
        q = torch.randn((NH, D), generator=gen).to(torch.float16)
        kc, ks = oq.kv_quantize_rows(torch.randn((NH * ctx, D), generator=gen).to(torch.float16).numpy())
        vc, vs = oq.kv_quantize_rows(torch.randn((NH * ctx, D), generator=gen).to(torch.float16).numpy())
        kc, vc = torch.from_numpy(kc).reshape(NH, ctx, D), torch.from_numpy(vc).reshape(NH, ctx, D)
        ks, vs = torch.from_numpy(ks).reshape(NH, ctx), torch.from_numpy(vs).reshape(NH, ctx)
        out["C3 KV-INT8 attention ctx %d" % ctx] = timeit(
            lambda: ops.int8_attention_folded(q, kc, ks, vc, vs, ctx).to(torch.float16))
    xn = ops.rms_norm(x.reshape(-1), gamma, s.eps)
    out["C4 RMSNorm 2048"] = timeit(lambda: ops.rms_norm(x.reshape(-1), gamma, s.eps))
    out["C4 qkv w8 GEMV 6144x2048"] = timeit(
        lambda: ops.dequant_gemm_separate(xn.reshape(1, -1), L0.qkv_codes, L0.qkv_scale, g, out_dtype=torch.float16))
    qkv = ops.dequant_gemm_separate(xn.reshape(1, -1), L0.qkv_codes, L0.qkv_scale, g, out_dtype=torch.float16)
    cos, sin = ops.rotary_cos_sin(torch.tensor([4096]), D, s.rope_theta)

    def qk_norm_rope():
        qn = ops.rms_norm(qkv[0, :HD], L0.q_norm, s.eps).reshape(NH, D)
        kn = ops.rms_norm(qkv[0, HD:2 * HD], L0.k_norm, s.eps).reshape(NH, D)
        ops.rope_fused(qn, cos[0], sin[0])
        ops.rope_fused(kn, cos[0], sin[0])

    out["C4 q/k RMSNorm + RoPE"] = timeit(qk_norm_rope)
    a = torch.randn((1, HD), generator=gen).to(torch.float16)
    out["C4 o_proj w8 GEMV 2048x2048"] = timeit(
        lambda: ops.dequant_gemm_separate(a, L0.o_codes, L0.o_scale, g, out_dtype=torch.float16))
    out["C4 lm_head w8 GEMV 50304x2048"] = timeit(
        lambda: ops.dequant_gemm_separate(xn.reshape(1, -1), host.lm_codes, host.lm_scale, g, out_dtype=torch.float16))
    for name, r in out.items():
        log("cpu op %-52s p50 %10.1f us  p99 %10.1f us" % (name, r["cpu_us_p50"], r["cpu_us_p99"]))
    return out


def attach_gpu_op_times(ops_cpu: dict, kt: dict, cfg: dict) -> dict:
    """The GPU microseconds (isolated, cold) of the kernels that compute each CPU operator."""
    def kavg(*names):
        try:
            return sum(kt[n]["avg_us"] for n in names)
        except KeyError:
            return None

    def cavg(prefix):
        for k, v in cfg.items():
            if k.startswith(prefix):
                return v["avg_us"]
        return None

    qkv = [k for k in kt if k.startswith("gemv_w8 qkv")]
    oproj = [k for k in kt if k.startswith("attn_merge_o_proj") or k.startswith("gemv_w8 o_proj")]
    router = [k for k in kt if k.startswith("router_logits")]
    lm = [k for k in kt if k.startswith("gemv_w8 lm_head")]
    gpu = {
        "C1": (kavg(*(router + ["moe_gate_up_w8_routed", "moe_down_w8"])),
               "router logits + routed gate/up + down launches"),
        "C2 split-KV fp16 attention ctx 1024": (cavg("attn_f16 ctx 1024"), "split + merge"),
        "C2 split-KV fp16 attention ctx 4096": (cavg("attn_f16 ctx 4096"), "split + merge"),
        "C3 KV-INT8 attention ctx 4096": (cavg("attn_i8 ctx 4096"), "split + merge"),
        "C3 KV-INT8 attention ctx 16384": (cavg("attn_i8 ctx 16384"), "split + merge"),
        "C4 RMSNorm 2048": (None, "fused into the qkv GEMV prologue"),
        "C4 qkv w8 GEMV 6144x2048": (kavg(*qkv), "qkv GEMV with the input RMSNorm in its prologue"),
        "C4 q/k RMSNorm + RoPE": (None, "fused into the attention launch"),
        "C4 o_proj w8 GEMV 2048x2048": (kavg(*oproj), "o_proj GEMV (with the attention merge when fused)"),
        "C4 lm_head w8 GEMV 50304x2048": (kavg(*lm), "lm_head GEMV + greedy argmax (2 launches)"),
    }
    for name, r in ops_cpu.items():
        key = "C1" if name.startswith("C1") else name
        us, what = gpu.get(key, (None, ""))
        r["gpu_us"] = us
        r["gpu_kernels"] = what
    return ops_cpu


# ---------------------------------------------------------------------------
def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------------
# The benchmark's attention configs as isolated kernels (fp16 and KV-INT8 split-KV)
# ---------------------------------------------------------------------------
def attention_configs(torch, hip, flusher, reps: int) -> dict:
    """Split-KV decode attention at the benchmark's shapes, cold, 16 layers' worth of
    caches per pass (split kernel + LSE merge, chunks of 256 cache slots):
    fp16 K/V at ctx 1024 and 4096, KV-INT8 at 4096 and 16384.  Algorithmic
    bytes: fp16 4 * 16 * ctx * 128; int8 4160 * ctx; plus q and partials."""
    dev = flusher.buf.device
    heads, D, copies = 16, 128, 16
    qk_scale = (1.0 / math.sqrt(D)) * 1.4426950408889634
    out = {}
    for kind, ctx in (("f16", 1024), ("f16", 4096), ("i8", 4096), ("i8", 16384)):
        ns = ctx // 256
        q = torch.randn((heads * D,), device=dev).to(torch.float16)
        filled = torch.tensor([ctx], dtype=torch.int32, device=dev)
        m = torch.empty((heads * ns,), dtype=torch.float32, device=dev)
        l = torch.empty_like(m)
        acc = torch.empty((heads * ns * D,), dtype=torch.float32, device=dev)
        o = torch.empty((heads * D,), dtype=torch.float16, device=dev)
        P, st = hip.ptr, hip.stream_of
        caches = []
        for _ in range(copies):
            if kind == "f16":
                caches.append([torch.randn((heads * ctx * D,), device=dev).to(torch.float16) for _ in range(2)])
            else:
                c = [torch.randint(-127, 128, (heads * ctx * D,), dtype=torch.int8, device=dev) for _ in range(2)]
                sc = [torch.full((heads * ctx,), 0.01, dtype=torch.float16, device=dev) for _ in range(2)]
                caches.append(c + sc)
        if kind == "f16":
            nbytes = 4 * heads * ctx * D + heads * D * 2 + heads * ns * (D + 2) * 4
            fns = [lambda c=c: (hip.call("lemoq_attn_split_f16", P(q), P(c[0]), P(c[1]), ctx * D, P(filled), heads, D,
                                         ns, qk_scale, P(m), P(l), P(acc), st()),
                                hip.call("lemoq_attn_merge", P(m), P(l), P(acc), heads, ns, D, P(o), st()))
                   for c in caches]
        else:
            nbytes = KV_BYTES_PER_TOKEN_LAYER * ctx + heads * D * 2 + heads * ns * (D + 2) * 4
            fns = [lambda c=c: (hip.call("lemoq_attn_split_i8", P(q), P(c[0]), P(c[2]), P(c[1]), P(c[3]), ctx * D, ctx,
                                         P(filled), heads, D, ns, qk_scale, P(m), P(l), P(acc), st()),
                                hip.call("lemoq_attn_merge", P(m), P(l), P(acc), heads, ns, D, P(o), st()))
                   for c in caches]
        # one untimed call first: a kernel's first launch in the process pays
        # one-time costs (19.0 against 9.4 us for the fp16 ctx-1024 config)
        fns[0]()
        r = time_cold(torch, flusher, fns, reps)
        name = "attn_%s ctx %d (split + merge, %d splits)" % (kind, ctx, ns)
        r["bytes"] = int(nbytes)
        r["gbs"] = nbytes / (r["avg_us"] * 1e-6) / 1e9
        out[name] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()}
        log("config %-44s %8.2f us avg  %7.1f GB/s" % (name, r["avg_us"], r["gbs"]))
        del caches, fns
        torch.cuda.synchronize()
    return out


def format_gemvs(torch, hip, flusher, reps: int) -> dict:
    """The decode GEMV over each weight format of the dense dequant operator
    (w8 / w8 asymmetric / w4 / w4 asymmetric / MXFP4), at the qkv, o_proj and
    lm_head shapes, and the grouped MoE on 8- and 4-bit experts, cold (16
    weight copies per pass, caches flushed), one token in, fp16 out.
    Algorithmic bytes: codes + scales (+ zero points) + activations in and out."""
    dev = flusher.buf.device
    K, copies = 2048, 16
    P, st = hip.ptr, hip.stream_of
    x = torch.randn((1, K), device=dev).to(torch.float16)
    out = {}
    for fname, fmt, bits, asym in (("w8", 0, 8, False), ("w8_asym", 1, 8, True), ("w4", 2, 4, False),
                                   ("w4_asym", 3, 4, True), ("mxfp4", 4, 4, False)):
        group = 32 if fmt == 4 else 128
        for shape, N in (("qkv", 6144), ("o_proj", 2048), ("lm_head", 50304)):
            ng = K // group
            row_bytes = K if bits == 8 else K // 2
            y = torch.empty((1, N), dtype=torch.float16, device=dev)
            ws = []
            for _ in range(copies):
                codes = torch.randint(0, 256, (N, row_bytes), dtype=torch.uint8, device=dev)
                if fmt == 4:
                    scale = torch.randint(118, 125, (N, ng), dtype=torch.uint8, device=dev)
                else:
                    scale = (torch.rand((N, ng), device=dev) * 0.01 + 1e-3).to(torch.float16)
                zero = torch.randint(0, 16, (N, ng), device=dev).to(torch.float16) if asym else None
                ws.append((codes, scale, zero))
            if fmt == 0:
                fns = [lambda c=c: hip.call("lemoq_gemv_w8", P(x), 1, K, P(c[0]), P(c[1]), N, K, group, P(y), 1, st())
                       for c in ws]
            else:
                fns = [lambda c=c: hip.call("lemoq_gemv_q", P(x), 1, K, P(c[0]), fmt, P(c[1]),
                                            P(c[2]) if c[2] is not None else None, 0, N, K, group, P(y), 1, st())
                       for c in ws]
            nbytes = N * row_bytes + N * ng * (1 if fmt == 4 else 2) * (2 if asym else 1) + K * 2 + N * 2
            fns[0]()
            r = time_cold(torch, flusher, fns, reps)
            name = "%s %s %dx%d" % (fname, shape, N, K)
            r["bytes"] = int(nbytes)
            r["gbs"] = nbytes / (r["avg_us"] * 1e-6) / 1e9
            r["frac_of_peak"] = r["gbs"] / HBM_PEAK_GBS
            out[name] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()}
            log("format %-28s %8.2f us avg  %7.1f GB/s" % (name, r["avg_us"], r["gbs"]))
            del ws, fns
            torch.cuda.synchronize()
    # the grouped MoE of one token at the OLMoE shape (64 experts, top-8, F 1024, H 2048),
    # 8-bit and 4-bit experts, ids given, 16 expert sets per pass
    E, F, H, top_k, group = 64, 1024, 2048, 8, 128
    ids = torch.randperm(E, device=dev)[:top_k].to(torch.int64)
    tw = torch.full((top_k,), 0.125, dtype=torch.float16, device=dev)
    xh = torch.randn((H,), device=dev).to(torch.float16)
    act = torch.empty((top_k, F), dtype=torch.float16, device=dev)
    yo = torch.empty((H,), dtype=torch.float16, device=dev)
    for bits in (8, 4):
        per = 8 // bits
        sets = []
        for _ in range(copies):
            dt = torch.int8 if bits == 8 else torch.uint8
            gu = torch.randint(-128 if bits == 8 else 0, 128 if bits == 8 else 256, (E, 2 * F, H // per), dtype=dt,
                               device=dev)
            dn = torch.randint(-128 if bits == 8 else 0, 128 if bits == 8 else 256, (E, H, F // per), dtype=dt,
                               device=dev)
            gs = (torch.rand((E, 2 * F, H // group), device=dev) * 0.01).to(torch.float16)
            ds = (torch.rand((E, H, F // group), device=dev) * 0.01).to(torch.float16)
            sets.append((gu, gs, dn, ds))
        gname, dname = ("lemoq_moe_gate_up_w8", "lemoq_moe_down_w8") if bits == 8 else (
            "lemoq_moe_gate_up_w4", "lemoq_moe_down_w4")
        for part, fn_of, nbytes in (
            ("gate_up", lambda c: (lambda: hip.call(gname, P(xh), P(c[0]), P(c[1]), P(ids), top_k, E, F, H, group,
                                                    P(act), st())),
             top_k * 2 * F * (H // per + (H // group) * 2) + H * 2 + top_k * F * 2),
            ("down", lambda c: (lambda: hip.call(dname, P(act), P(c[2]), P(c[3]), P(ids), P(tw), top_k, E, H, F, group,
                                                 None, P(yo), st())),
             top_k * H * (F // per + (F // group) * 2) + top_k * F * 2 + H * 2)):
            fns = [fn_of(c) for c in sets]
            fns[0]()
            r = time_cold(torch, flusher, fns, reps)
            name = "w%d moe %s (%d of %d experts)" % (bits, part, top_k, E)
            r["bytes"] = int(nbytes)
            r["gbs"] = nbytes / (r["avg_us"] * 1e-6) / 1e9
            r["frac_of_peak"] = r["gbs"] / HBM_PEAK_GBS
            out[name] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()}
            log("format %-28s %8.2f us avg  %7.1f GB/s" % (name, r["avg_us"], r["gbs"]))
        del sets
        torch.cuda.synchronize()
    return out


# HBM traffic from two rocprofv3 --pmc passes
# ---------------------------------------------------------------------------
COPY_BYTES = 512 << 20  # calibration copy: larger than the 256 MB Infinity Cache


def synthetic_cache(torch, sess, filled: int, seed: int = 7) -> None:
    """Random KV-INT8 contents (codes in [-127, 127], scales in [0.01, 0.02)) and
    the decode position at ``filled`` - 1, in place of a prefill: the isolated
    kernels' bytes and times depend on the filled length, not on the values."""
    g = torch.Generator(device=sess.device).manual_seed(seed)
    for kv in sess.kv:
        for n in ("kc", "vc"):
            kv[n].random_(-127, 128, generator=g)
        for n in ("ks", "vs"):
            kv[n].uniform_(0.01, 0.02, generator=g)
    sess.set_position(filled - 1, token=1)
    torch.cuda.synchronize()


def copy_calibration(torch, hip, flusher, reps: int = 2) -> dict:
    """``reps`` cold copies of COPY_BYTES with lemoq_copy_probe (each byte read once and
    written once): the profiler's FETCH_SIZE / WRITE_SIZE of these dispatches
    calibrate the same counters on the step's kernels."""
    dst = torch.empty((COPY_BYTES,), dtype=torch.uint8, device=flusher.buf.device)
    for _ in range(reps):
        flusher.flush()
        hip.call("lemoq_copy_probe", hip.ptr(flusher.buf), hip.ptr(dst), COPY_BYTES, 4096, hip.stream_of())
    torch.cuda.synchronize()
    return {"copy_bytes": COPY_BYTES, "copies": reps, "flush_bytes": flusher.nbytes}


def _pmc_rows(path: str, counter: str) -> list:
    """(dispatch id, kernel name, value) of one counter from a rocprofv3 counter_collection csv, in dispatch order."""
    import csv

    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") != counter:
                continue
            rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return rows


def summarize_pmc(fetch_csv: str, write_csv: str, plan_json: str, out_dir: str) -> dict:
    """Per-kernel HBM bytes per launch from a FETCH_SIZE pass and a WRITE_SIZE pass
    (KiB per dispatch) of ``bench.py --mode traffic``.  Each counter is scaled
    by bytes / counter of the calibration copy (read COPY_BYTES, wrote
    COPY_BYTES).  The traffic-mode dispatches of the plan's kernels are matched
    to its kernel table in order (cache flushes and torch's own copies and
    fills in between are skipped), and every matched kernel name is checked
    against the plan."""
    with open(plan_json) as f:
        plan = json.loads(f.read().strip().splitlines()[-1])
    passes = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = _pmc_rows(path, counter)
        copies = [v for _, n, v in rows if "copy_probe_kernel" in n]
        flushes = [v for _, n, v in rows if "read_probe_kernel" in n]
        if len(copies) < 1:
            raise SystemExit("%s: no copy_probe_kernel dispatch in %s" % (counter, path))
        kib = sum(copies) / len(copies)
        factor = plan["calibration"]["copy_bytes"] / (kib * 1024.0)
        first_copy = next(i for i, (_, n, _) in enumerate(rows) if "copy_probe_kernel" in n)
        known = {kn for k in plan["kernels"].values() for kn in k["dispatch_kernels"]}
        seq = [(n, v) for _, n, v in rows[first_copy:] if any(kn in n for kn in known)]
        per = {}
        i = 0
        for name, k in plan["kernels"].items():
            calls = k["launches"]
            vals = []
            for _ in range(calls):
                tot = 0.0
                for kn in k["dispatch_kernels"]:
                    if i >= len(seq) or kn not in seq[i][0]:
                        got = seq[i][0] if i < len(seq) else "end of trace"
                        raise SystemExit("%s: dispatch %d is %r, the plan expects %s" % (counter, i, got, kn))
                    tot += seq[i][1]
                    i += 1
                vals.append(tot)
            per[name] = sum(vals) / len(vals) * 1024.0 * factor
        passes[counter] = {"factor": factor, "copy_kib": kib,
                           "flush_kib": sum(flushes) / len(flushes) if flushes else None, "per": per}
    out = {"calibration": {
        "copy_bytes": plan["calibration"]["copy_bytes"],
        "fetch_factor": passes["FETCH_SIZE"]["factor"], "write_factor": passes["WRITE_SIZE"]["factor"],
        "copy_fetch_kib": passes["FETCH_SIZE"]["copy_kib"], "copy_write_kib": passes["WRITE_SIZE"]["copy_kib"],
        "flush_fetch_kib": passes["FETCH_SIZE"]["flush_kib"], "flush_bytes": plan["calibration"]["flush_bytes"],
    }, "ctx": plan["ctx"]}
    lines = ["| kernel | algorithmic B/launch | HBM read B | HBM write B | traffic / algorithmic |", "|---|---|---|---|---|"]
    for name, k in plan["kernels"].items():
        rd, wr = passes["FETCH_SIZE"]["per"][name], passes["WRITE_SIZE"]["per"][name]
        out[name] = {"traffic_bytes": int(round(rd + wr)), "read_bytes": int(round(rd)), "write_bytes": int(round(wr)),
                     "algorithmic_bytes": k["bytes"], "launches": k["launches"]}
        lines.append("| %s | %d | %d | %d | %.3f |" % (name, k["bytes"], rd, wr, (rd + wr) / k["bytes"]))
    os.makedirs(out_dir, exist_ok=True)
    with open(os.path.join(out_dir, "traffic.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    return {"table": "\n".join(lines), "data": out}


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.summarize_pmc:
        r = summarize_pmc(*args.summarize_pmc, out_dir=args.profiles_dir)
        print(r["table"])
        return 0
    if args.summarize_prefill:
        print(summarize_prefill(args.summarize_prefill, args.ctx))
        return 0
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace))
        return 0
    if args.summarize_step:
        print(summarize_step(args.summarize_step, last=args.summarize_last))
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the batch-1 decode "
              "step runs on one MI355X); run with --gpus 1", file=sys.stderr)
        return 2
    import torch

    from lemoq import _hip
    from lemoq.model.olmoe import OLMOE_1B_7B, OlmoeW8Weights

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    _hip.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log("device %s, %d CUs" % (torch.cuda.get_device_name(dev), torch.cuda.get_device_properties(dev).multi_processor_count))
    t = time.time()
    w = OlmoeW8Weights.random(OLMOE_1B_7B, seed=args.seed, device=dev)
    torch.cuda.synchronize()
    log("weights ready %.1fs (%.1f MB streamed per token)" % (time.time() - t, w.shape.weight_bytes_per_token() / 1e6))
    flusher = Flusher(torch, _hip, dev)
    read_bw = flusher.read_bandwidth_gbs()
    log("measured read bandwidth %.1f GB/s" % read_bw)

    if args.mode == "traffic":
        from lemoq.model.olmoe import DecodeSession

        sess = DecodeSession(w, [1] * args.ctx, max_new_tokens=2, kv_cache="int8")
        synthetic_cache(torch, sess, sess.ctx + 1)
        cal = copy_calibration(torch, _hip, flusher)
        kt = kernel_table(torch, _hip, w, sess, flusher, args.kernel_reps, floors=False)
        print(json.dumps({"mode": "traffic", "ctx": args.ctx, "calibration": cal, "kernels": kt}))
        return 0

    if args.mode == "step":
        from lemoq.model.olmoe import DecodeSession, OlmoeW8Weights

        w4 = args.weights == "w4a16"
        if w4:
            del w
            torch.cuda.empty_cache()
            w = OlmoeW8Weights.random(OLMOE_1B_7B, seed=args.seed, device=dev, bits=4, lm_head="fp16")
        sess = DecodeSession(w, [1] * args.ctx, max_new_tokens=args.warmup + args.steps + 1, kv_cache=args.kv_cache)
        sess.capture()
        sess.prefill()
        sess.replay(args.warmup)
        t0 = time.perf_counter()
        sess.replay(args.steps)
        ms = (time.perf_counter() - t0) * 1e3 / args.steps
        log("ctx %d: %d replays, %.4f ms/token" % (args.ctx, args.steps, ms))
        print(json.dumps({"mode": "step", "ctx": args.ctx, "kv_cache": args.kv_cache, "weights": args.weights,
                          "steps": args.steps, "ms_per_token": ms, "launches_per_step": sess.launches_per_step}))
        return 0

    if args.mode == "prefill":
        from lemoq.model.olmoe import DecodeSession

        res = {"mode": "prefill"}
        for ctx in [c for c in (args.ctx, args.ctx2) if c]:
            sess = DecodeSession(w, [1] * ctx, max_new_tokens=2, kv_cache="int8")
            sess.capture()
            res["ctx%d" % ctx] = measure_prefill(torch, sess)
            log("ctx %d: TTFT p50 %.3f ms" % (ctx, res["ctx%d" % ctx]["p50"]))
            del sess
        print(json.dumps(res))
        return 0

    if args.mode == "kernels":
        from lemoq.model.olmoe import DecodeSession

        sess = DecodeSession(w, [1] * args.ctx, max_new_tokens=2, kv_cache="int8")
        sess.capture()
        sess.prefill()
        kt = kernel_table(torch, _hip, w, sess, flusher, args.kernel_reps)
        print(json.dumps({"mode": "kernels", "read_bw_gbs": read_bw, "kernels": kt}))
        return 0

    check_n = 0 if args.no_cpu else max(1, args.cpu_check_steps)
    sess, r1 = time_decode(torch, w, args.ctx, args.steps, args.warmup, check_n)
    snap = None
    check_tokens: list[int] = []
    check_logits = []
    if check_n:
        snap = (sess.kv_cpu(), int(sess.token.item()), sess.position)
        p0 = sess.position
        for _ in range(check_n):
            sess.replay(1)
            check_logits.append(sess.logits_cpu())
        check_tokens = [int(t) for t in sess.history[p0 + 1: p0 + 1 + check_n].tolist()]
    kt = kernel_table(torch, _hip, w, sess, flusher, args.kernel_reps)
    cfg = attention_configs(torch, _hip, flusher, args.kernel_reps)
    fmts = None if args.no_formats else format_gemvs(torch, _hip, flusher, args.kernel_reps)
    kv16 = None
    if not args.no_kv_fp16:
        del sess  # its caches: the fp16-cache sessions take their own
        sess = None
        kv16 = {str(c): time_kv_fp16(torch, w, c, args.steps, args.warmup, read_bw)
                for c in (args.ctx, args.ctx2) if c}
    w4a16 = None
    if not args.no_w4a16:
        del sess
        sess = None
        w4a16 = {str(c): time_w4a16(torch, OLMOE_1B_7B, args.seed, dev, c, args.steps, args.warmup, read_bw)
                 for c in (args.ctx, args.ctx2) if c}
    del sess
    r2 = None
    snap2 = None
    if args.ctx2:
        s2, r2 = time_decode(torch, w, args.ctx2, args.steps, args.warmup, 0)
        if check_n:
            snap2 = (s2.kv_cpu(), int(s2.token.item()), s2.position)
        del s2
    torch.cuda.synchronize()

    cpu = None
    if check_n:
        host = w.to_host()
        cpu = cpu_baseline(torch, host, snap, check_tokens, check_logits, warmup=args.cpu_warmup,
                           timed=args.cpu_timed, timed_1t=args.cpu_timed_1t, snap2=snap2)
        if not args.no_cpu_ops:
            cpu["ops"] = attach_gpu_op_times(
                cpu_ops_baseline(torch, host, warmup=args.cpu_warmup, timed=args.cpu_timed, seed=args.seed), kt, cfg)
        del host

    dom_name = "moe_gate_up_w8_routed"
    dom = kt[dom_name]
    traffic = _traffic_from_profiles(dom_name)
    in_graph_us = _in_graph_from_profiles(DOM_DISPATCH)
    line = {
        "metric": METRIC,
        "value": r1["ms_per_token_repeats_p50"],
        "unit": "ms/token",
        "stat": "p50 over 3 repeats of the wall-clock mean of 32 graph replays, each repeat from the same "
                "prefilled state (the reference's measure_graph_gap, benchmarks/cudagraph.py:420-495, and its "
                "per-token p50, benchmarks/runner.py:984); step_ms_p50/p99 are per-step times with an event "
                "between replays",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r1["ms_per_token_repeats_p50"],
        "ms_per_step_mean": r1["ms_per_token"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": "OLMoE-1B-7B-shaped batch-1 greedy decode step (16 layers, hidden 2048, 16x128 heads, "
                        "64 experts top-8, ffn 1024, vocab 50304), w8a16 g128 + W8 lm_head + KV-INT8, "
                        "prompt %d x token 1, seeded random init, one hipGraph replay per token" % args.ctx,
            "ctx": args.ctx,
            "weights": "int8 per-group-128 codes, fp16 scales; fp32 accumulation",
        },
        "tokens_per_s": 1000.0 / r1["ms_per_token_repeats_p50"],
        "device_ms_per_token": r1["device_ms_per_token"],
        "host_share": r1["host_share"],
        "launches_per_step": r1["launches_per_step"],
        "step_bytes": r1["step_bytes"],
        "step_hbm_frac_of_peak": r1["step_bytes"] / (r1["device_ms_per_token"] * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "step_hbm_frac_of_measured": r1["step_bytes"] / (r1["device_ms_per_token"] * 1e-3) / 1e9 / read_bw,
        "measured_read_bw_gbs": read_bw,
        "reference_rtx5090_ms_per_token": REFERENCE_RTX5090_MS,
        "roofline": {
            "kernel": dom_name,
            "bound": "hbm",
            "achieved": dom["gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": dom["gbs"] / HBM_PEAK_GBS,
            "traffic": traffic,
            "bytes_per_launch": dom["bytes"],
            "avg_us": dom["avg_us"],
            # a launch that only reads the same bytes, timed the same way (cold, 64 launches)
            "read_floor_avg_us": kt[READ_FLOOR]["avg_us"],
            "frac_of_read_floor": kt[READ_FLOOR]["avg_us"] / dom["avg_us"],
            # the same kernel as it runs inside the step's graph replays
            "in_graph_avg_us": in_graph_us,
            "frac_in_graph": (dom["bytes"] / (in_graph_us * 1e-6) / 1e9 / HBM_PEAK_GBS) if in_graph_us else None,
            "in_graph_source": BENCH_TRACE + " (rocprofv3 --kernel-trace of this bench command)" if in_graph_us else None,
        },
        "kernels": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()
                        if kk != "dispatch_kernels"} for k, v in kt.items()},
    }
    line["attention_configs"] = cfg
    if fmts is not None:
        line["weight_formats"] = fmts
    from lemoq.kernels.fusion_switches import fusion_payload_fields  # noqa: PLC0415

    # the reference records its switches in every payload; here all are the fused form, and the
    # headline runs the KV-INT8 cache whatever LEMOQ_KV_INT8 says (the fp16 cache is `kv_fp16`)
    line["fusion_switches"] = fusion_payload_fields()
    if kv16 is not None:
        kv16["reference_rtx5090_ms_per_token"] = REFERENCE_RTX5090_KV_F16_MS
        kv16["what"] = ("the same step over the fp16 cache (DecodeSession(kv_cache='fp16'): the reference's cell "
                        "with KV-INT8 off), prompt ctx x token 1, timed as the headline")
        line["kv_fp16"] = kv16
    if w4a16 is not None:
        w4a16["what"] = ("the reference's w4a16 cell on the same shape: attention and experts as 4-bit symmetric RTN "
                         "codes (g128), router and lm_head fp16, KV-INT8 (OlmoeW8Weights.random(bits=4, "
                         "lm_head='fp16')); batched prefill of ctx x token 1 (TTFT beside it), timed as the "
                         "headline; the reference publishes no w4a16 latency (its accuracy gate fails, "
                         "RESULTS.md:166)")
        line["w4a16"] = w4a16
    line["step_ms_p50"], line["step_ms_p99"] = r1["step_ms_p50"], r1["step_ms_p99"]
    gk = "ms_per_token_graph%d" % MULTI_STEPS
    line[gk] = r1[gk]  # MULTI_STEPS steps per graph launch (not the headline)
    line["prefill"] = _prefill_summary(r1, r2)
    # the reference's repeated timing: 3 repeats x >= 20 replays from the same prefilled state
    line["repeats"] = {"ctx%d" % r["ctx"]: r["repeats"] for r in (r1, r2) if r is not None}
    line["graph_gate"] = {"ctx%d" % r["ctx"]: r["graph_gate"] for r in (r1, r2) if r is not None}
    if r2 is not None:
        line["ctx2"] = r2
        # the headline statistic at the second context
        line["ms_per_token_ctx%d" % args.ctx2] = r2["ms_per_token_repeats_p50"]
        line["step_ms_p50_ctx%d" % args.ctx2] = r2["step_ms_p50"]
        line["ms_per_token_mean_ctx%d" % args.ctx2] = r2["ms_per_token"]
        line["step_hbm_frac_of_peak_ctx%d" % args.ctx2] = (
            r2["step_bytes"] / (r2["device_ms_per_token"] * 1e-3) / 1e9 / HBM_PEAK_GBS)
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line))
    sys.stdout.flush()
    return 0


# Launch order of one batched prefill (lemoq.model.prefill.prefill_prompt):
# gather, layer 0's input norm, 15 x [11 launches] (each combine also writes the
# next layer's input norm), the last layer (qkv and KV rows for every position,
# then 10 launches on the last row), the lm_head GEMV of the last row
# (final norm in its prologue), then the greedy pick; each role with the
# kernel-name fragment its dispatch must carry.
PREFILL_HEAD_ROLES = (("gather_rows", "gather_rows_kernel"), ("rmsnorm (input, layer 0)", "rmsnorm_kernel"))
PREFILL_LAYER_ROLES = (("gemm_w8 qkv", "gemm_kernel<true"),
                       ("qk_rows (q/k norm, RoPE, KV-INT8)", "qk_rows_kernel"), ("attn_prefill", "attn_prefill_kernel"),
                       ("gemm_w8 o_proj (+residual)", "gemm_kernel<true"), ("rmsnorm (post-attention)", "rmsnorm_kernel"),
                       ("gemm_f16 router (split-K partials)", "gemm_kernel<false"),
                       ("route_topk (+ split-K sum)", "route_topk_kernel"),
                       ("moe_prefill_sort", "moe_sort_kernel"), ("moe_prefill_gate_up", "moe_gate_up_kernel"),
                       ("moe_prefill_down", "moe_down_kernel"))
PREFILL_COMBINE_NORM = ("moe_prefill_combine (+residual, next input norm)", "moe_combine_kernel<true")
# the last layer: its qkv and KV rows for every position, the rest for the last row only
PREFILL_LAST_LAYER_ROLES = (("gemm_w8 qkv", "gemm_kernel<true"),
                            ("qk_rows (q/k norm, RoPE, KV-INT8)", "qk_rows_kernel"),
                            ("last row: attention split-KV", "attn_split_kernel"),
                            ("last row: attention merge", "attn_merge"),
                            ("last row: o_proj (+residual)", "gemm_kernel<true"),
                            ("last row: post norm", "rmsnorm_kernel"),
                            ("last row: router (split-K partials)", "gemm_kernel<false"),
                            ("last row: route_topk", "route_topk_kernel"),
                            ("last row: moe sort", "moe_sort_kernel"),
                            ("last row: moe gate_up", "moe_gate_up_kernel"),
                            ("last row: moe down", "moe_down_kernel"),
                            ("last row: moe combine (+residual)", "moe_combine_kernel<false"))
PREFILL_TAIL_ROLES = (("gemv_w8 lm_head (last row, + final norm)", "gemv_w8_kernel"),
                      ("argmax_advance", "argmax_advance_kernel"))


def prefill_roles(n_layers: int = 16) -> list:
    roles = list(PREFILL_HEAD_ROLES)
    for _ in range(n_layers - 1):
        roles += list(PREFILL_LAYER_ROLES)
        roles.append(PREFILL_COMBINE_NORM)
    return roles + list(PREFILL_LAST_LAYER_ROLES) + list(PREFILL_TAIL_ROLES)


def prefill_flops(role: str, T: int, shape=None) -> float:
    """Algorithmic FLOPs of one launch of a prefill role at prompt length T (OLMoE-1B-7B)."""
    H, NH, D, E, K, F, V = 2048, 16, 128, 64, 8, 1024, 50304
    return {
        "gemm_w8 qkv": 2.0 * T * 3 * NH * D * H,
        "gemm_w8 o_proj (+residual)": 2.0 * T * H * NH * D,
        "gemm_f16 router (split-K partials)": 2.0 * T * E * H,
        "attn_prefill": 4.0 * NH * D * T * (T + 1) / 2,
        "moe_prefill_gate_up": 2.0 * T * K * 2 * F * H,
        "moe_prefill_down": 2.0 * T * K * H * F,
        "gemv_w8 lm_head (last row, + final norm)": 2.0 * V * H,
    }.get(role, 0.0)


def summarize_prefill(trace_csv: str, ctx: int) -> str:
    """Markdown table of the prefills found in a rocprofv3 kernel trace: each prefill
    starts at a gather_rows dispatch; roles follow PREFILL_LAYER_ROLES."""
    import csv as _csv

    # the library's own dispatches only (torch's fills and copies run between them)
    rows = sorted((r for r in _csv.DictReader(open(trace_csv))
                   if not r["Kernel_Name"].startswith("__amd_rocclr") and "at::native" not in r["Kernel_Name"]),
                  key=lambda r: int(r["Start_Timestamp"]))
    starts = [i for i, r in enumerate(rows) if "gather_rows_kernel" in r["Kernel_Name"]]
    per_role: dict = {}
    roles = prefill_roles(16)
    total = []
    for st in starts:
        seq = rows[st: st + len(roles)]
        if len(seq) < len(roles):
            continue
        for (role, frag), r in zip(roles, seq):
            if frag not in r["Kernel_Name"]:
                raise ValueError("prefill launch order changed: %r where %s (%s) was expected"
                                 % (r["Kernel_Name"][:80], role, frag))
            per_role.setdefault(role, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
        total.append((int(seq[-1]["End_Timestamp"]) - int(seq[0]["Start_Timestamp"])) * 1e-3)
    n = len(total)
    if not n:
        return "no complete prefill found in %s" % trace_csv
    out = ["| role | launches per prefill | avg us | ms per prefill | share %% | GFLOP per launch | TF/s | %% of %.0f TF/s |"
           % MFMA_F16_PEAK_TFLOPS, "|---|---|---|---|---|---|---|---|"]
    span = sum(total) / n
    busy = sum(sum(v) for v in per_role.values()) / n
    for role, v in sorted(per_role.items(), key=lambda kv: -sum(kv[1])):
        launches = len(v) // n
        avg = sum(v) / len(v)
        fl = prefill_flops(role, ctx)
        tf = fl / (avg * 1e-6) / 1e12 if fl else 0.0
        out.append("| %s | %d | %.2f | %.3f | %.1f | %s | %s | %s |" % (
            role, launches, avg, sum(v) / n / 1e3, 100.0 * sum(v) / n / busy, "%.2f" % (fl / 1e9) if fl else "-",
            "%.1f" % tf if fl else "-", "%.1f" % (100 * tf / MFMA_F16_PEAK_TFLOPS) if fl else "-"))
    out.append("")
    out.append("%d prefills of %d tokens; kernel time %.3f ms per prefill, first launch start to last launch "
               "end %.3f ms (the gaps are launch and host overhead)." % (n, ctx, busy / 1e3, span / 1e3))
    return "\n".join(out)


def _short_kernel(name: str) -> str:
    n = name.replace("(anonymous namespace)::", "").replace("void ", "")
    n = n.split("(")[0] if "<" not in n else n[: n.rfind(">") + 1]
    return n


def summarize_trace(trace_csv: str) -> str:
    """Per-kernel durations of a rocprofv3 kernel trace of a full bench run, split
    into the cold isolated launches of the kernel table and all other launches
    (the graph replays and prefills).  A kernel-table pass is the run of
    dispatches after a cache flush (``read_probe_kernel``) made of the first two
    kernel names of the run (one kernel, or a kernel pair such as lm_head +
    argmax or split + merge); the flushes of the bandwidth probe, followed by a
    prefill (``gather_rows_kernel``), start no pass."""
    import csv as _csv

    rows = sorted((r for r in _csv.DictReader(open(trace_csv))
                   if not r["Kernel_Name"].startswith("__amd_rocclr") and "at::native" not in r["Kernel_Name"]),
                  key=lambda r: int(r["Start_Timestamp"]))
    iso = set()
    for i, r in enumerate(rows):
        if "read_probe_kernel" not in r["Kernel_Name"] or i + 1 >= len(rows):
            continue
        first = rows[i + 1]["Kernel_Name"]
        if "read_probe_kernel" in first or "gather_rows_kernel" in first:
            continue
        names = {first}
        if i + 2 < len(rows) and "read_probe_kernel" not in rows[i + 2]["Kernel_Name"]:
            names.add(rows[i + 2]["Kernel_Name"])
        j = i + 1
        while j < len(rows) and rows[j]["Kernel_Name"] in names:
            iso.add(j)
            j += 1
    stats: dict = {}
    for i, r in enumerate(rows):
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
        e = stats.setdefault(_short_kernel(r["Kernel_Name"]), {"graph": [], "iso": []})
        e["iso" if i in iso else "graph"].append(d)
    out = ["| kernel | in-graph / other launches | avg us | isolated cold launches | avg us |", "|---|---|---|---|---|"]
    for name, e in sorted(stats.items(), key=lambda kv: -(sum(kv[1]["graph"]) + sum(kv[1]["iso"]))):
        g, c = e["graph"], e["iso"]
        out.append("| %s | %d | %s | %d | %s |" % (name[:100], len(g), "%.2f" % (sum(g) / len(g)) if g else "-",
                                                    len(c), "%.2f" % (sum(c) / len(c)) if c else "-"))
    return "\n".join(out)


# The decode step's kernels in launch order (csrc/step.hip): per layer, then the lm_head pair.
STEP_LAYER_KERNELS = [
    ("qkv (+ input RMSNorm)", "gemv_w8_kernel<2, 2, 0, true>"),
    ("attention split (+ q/k norm, RoPE, cache write)", "attn_split_fused_"),  # the _i8 or _f16 kernel
    ("merge + o_proj", "merge_oproj_kernel"),
    ("residual + norm + router", "router_resid_kernel"),
    ("gate/up (+ routing)", "moe_gate_up_kernel<2, 2, 1, true>"),
    ("down (+ residual)", "moe_down_kernel<1, 4, true>"),
]
STEP_TAIL_KERNELS = [("lm_head (+ final norm, argmax partials)", "gemv_w8_kernel<2, 2, 1, true>"),
                     ("argmax + advance", "argmax_advance_kernel<true")]  # <true, false>: over the partials


# The 4-bit step (--weights w4a16) at the OLMoE shape by position: per layer the 6
# launches below (layer 0's q|k|v GEMV gathers the embedding row), then the fp16
# lm_head with the argmax partials and the greedy pick over them.  A trace of it
# is recognised by its fp16 lm_head kernel.
STEP_W4_LAYER = ["qkv (4-bit, + input RMSNorm)", "attention split (+ q/k norm, RoPE, cache write)",
                 "merge + o_proj (4-bit)", "residual + norm + router",
                 "gate/up (4-bit, + routing)", "down (4-bit, + residual)"]
STEP_W4_HEAD = ["lm_head fp16 (+ final norm, argmax partials)", "argmax + advance"]
STEP_W4_MARK = "lm_head_f16_argmax_kernel<"
STEP_W4_END = "argmax_advance_kernel<true"  # over the partials


def _w4_roles() -> list:
    """Role of each launch of a whole 4-bit step, by position."""
    return STEP_W4_LAYER * 16 + STEP_W4_HEAD


def summarize_step(trace_csv: str, last: int = 0) -> str:
    """Per-kernel durations of the decode step's graph replays in a rocprofv3
    kernel trace of ``bench.py --mode step``, and the step's timeline: each step
    is the run of the step's kernels ending with the argmax launch; its span is
    first start to last end, its busy time the sum of its kernels' durations,
    and the rest of the span is the time between kernels (launch and dispatch
    gaps inside the graph).  ``last`` keeps only the last N whole steps (the
    4-bit step's prompt is fed through the step itself).  A trace of the 4-bit
    step (``--weights w4a16``) is recognised by its fp16 lm_head kernel."""
    import csv as _csv

    all_rows = list(_csv.DictReader(open(trace_csv)))
    if any(STEP_W4_MARK in _short_kernel(r["Kernel_Name"]) for r in all_rows):
        return _summarize_step_w4(all_rows, last, trace_csv)
    names = [k for _, k in STEP_LAYER_KERNELS + STEP_TAIL_KERNELS]
    rows = sorted((r for r in all_rows if any(n in _short_kernel(r["Kernel_Name"]) for n in names)),
                  key=lambda r: int(r["Start_Timestamp"]))
    steps, cur = [], []
    for r in rows:
        cur.append(r)
        if "argmax_advance_kernel<true" in _short_kernel(r["Kernel_Name"]):
            steps.append(cur)
            cur = []
    per_step = len(STEP_LAYER_KERNELS) * 16 + len(STEP_TAIL_KERNELS)
    steps = [st for st in steps if len(st) == per_step]  # whole 16-layer steps only (the prefill's seed pick is not)
    if last > 0:
        steps = steps[-last:]
    if not steps:
        return "no whole decode steps in %s" % trace_csv
    labels = [lbl for lbl, _ in STEP_LAYER_KERNELS + STEP_TAIL_KERNELS]

    def role(i, r):
        return next(lbl for lbl, k in STEP_LAYER_KERNELS + STEP_TAIL_KERNELS if k in _short_kernel(r["Kernel_Name"]))

    return _step_table(steps, per_step, labels, role)


def _summarize_step_w4(all_rows: list, last: int, trace_csv: str) -> str:
    """``summarize_step`` of the 4-bit step: every dispatch between two greedy
    picks is one step (the graph holds nothing else), roles by position."""
    rows = sorted(all_rows, key=lambda r: int(r["Start_Timestamp"]))
    steps, cur = [], []
    for r in rows:
        cur.append(r)
        if STEP_W4_END in _short_kernel(r["Kernel_Name"]):
            steps.append(cur)
            cur = []
    roles = _w4_roles()
    per_step = len(roles)
    # a chunk may start with other dispatches before the step (the first one after
    # the session's set-up, or a batched prefill): keep its last per_step launches
    # when they open with the q|k|v GEMV (layer 0 gathers the embedding row inside
    # it) and close with the fp16 lm_head and the pick
    steps = [st[-per_step:] for st in steps
             if len(st) >= per_step and "gemv_q_kernel<" in _short_kernel(st[-per_step]["Kernel_Name"])
             and STEP_W4_MARK in _short_kernel(st[-2]["Kernel_Name"])]
    if last > 0:
        steps = steps[-last:]
    if not steps:
        return "no whole 4-bit decode steps in %s" % trace_csv
    labels = STEP_W4_LAYER + STEP_W4_HEAD
    return _step_table(steps, per_step, labels, lambda i, r: roles[i])


def _step_table(steps: list, per_step: int, labels: list, role) -> str:
    dur: dict = {}
    spans, busy = [], []
    for st in steps:
        t0, t1 = int(st[0]["Start_Timestamp"]), int(st[-1]["End_Timestamp"])
        spans.append((t1 - t0) * 1e-3)
        b = 0.0
        for i, r in enumerate(st):
            d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
            b += d
            dur.setdefault(role(i, r), []).append(d)
        busy.append(b)
    spans.sort()
    busy.sort()
    n = len(steps)
    out = ["%d whole steps of %d launches; step span p50 %.1f us (min %.1f, max %.1f); kernel busy time p50 %.1f us, "
           "so %.1f us (%.0f%%) of the span lies between kernels" % (
               n, per_step, spans[n // 2], spans[0], spans[-1], busy[n // 2], spans[n // 2] - busy[n // 2],
               100.0 * (spans[n // 2] - busy[n // 2]) / spans[n // 2]), "",
           "| kernel | launches per step | avg us | p50 us | min us | max us | us per step |", "|---|---|---|---|---|---|---|"]
    tot = 0.0
    for lbl in labels:
        v = sorted(dur.get(lbl, []))
        if not v:
            continue
        per = len(v) // n
        avg = sum(v) / len(v)
        tot += avg * per
        out.append("| %s | %d | %.2f | %.2f | %.2f | %.2f | %.1f |" % (lbl, per, avg, v[len(v) // 2], v[0], v[-1],
                                                                       avg * per))
    out.append("| **sum of kernel averages** | %d | | | | | %.1f |" % (per_step, tot))
    return "\n".join(out)


def _prefill_summary(*runs) -> dict:
    """TTFT p50 and E2E(N) = TTFT + N x per-token (the reference's composition,
    RESULTS.md:133-141) per context, beside the reference's published values."""
    out = {}
    for r in runs:
        if r is None:
            continue
        c = str(r["ctx"])
        ttft = r["ttft"]["p50"]
        out["ctx" + c] = {
            "ttft_ms_p50": ttft,
            "ttft_ms_min": r["ttft"]["min"],
            "ttft_ms_p50_random_prompt": r["ttft_random_prompt"]["p50"],
            "e2e_32_ms": ttft + 32 * r["ms_per_token"],
            "e2e_128_ms": ttft + 128 * r["ms_per_token"],
            "reference_rtx5090_ttft_ms": REFERENCE_RTX5090_TTFT_MS.get(c),
            "reference_rtx5090_e2e_32_ms": REFERENCE_RTX5090_E2E32_MS.get(c),
        }
    return out


# The roofline kernel's dispatch name in a rocprofv3 kernel trace.
DOM_DISPATCH = "moe_gate_up_kernel<2, 2, 1, true>"
BENCH_TRACE = os.path.join("profiles", "bench_kernel_trace.md")


def _in_graph_from_profiles(dispatch: str):
    """Average duration (us) of ``dispatch`` inside the graph replays, from the
    committed rocprofv3 kernel trace of this bench command (the table written by
    ``--summarize-trace``), or None.  Events time a whole replay, not one of its
    nodes, so the in-graph duration of one kernel comes from the profiler."""
    try:
        with open(os.path.join(REPO, BENCH_TRACE)) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) == 5 and cells[0] == dispatch and cells[2] != "-":
                    return float(cells[2])
    except (OSError, ValueError):
        pass
    return None


def _traffic_from_profiles(kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 --pmc summary, if present."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data.get(kernel, {}).get("traffic_bytes")
    except (OSError, ValueError):
        return None


if __name__ == "__main__":
    sys.exit(main())
