#!/usr/bin/env python3
"""Decode-step benchmark of the lemoq MI355X build (one GPU).

Workload: the OLMoE-1B-7B-shaped batch-1 decode step of the reference's
canonical cell (w8a16 g128 attention + experts, W8 lm_head, KV-INT8 cache,
split-KV attention, one graph per step): seeded random weights, prompt of
``ctx`` copies of token id 1, then greedy decode steps replayed from one
captured hipGraph.  The reference quotes this as ms/token at ctx 1024 and 4096
(README_EN.md:66-71 of LeanMoE-Quant, RTX 5090).

Printed: ONE JSON line on stdout.  ``value`` is ms/token at ``--ctx`` (wall
clock over exactly ``--steps`` replays, synchronised on both sides, after
``--warmup`` replays); the line also carries the second context, the step's
HBM roofline fraction, per-kernel cold timings, the dominant kernel's roofline
(``roofline``), the CPU oracle's ms/token on this host (``cpu_baseline``) and,
per context, the batched prefill's TTFT with E2E-32/128 beside the
reference's published values (``prefill``).  Progress goes to stderr.

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
    ap.add_argument("--cpu-budget-s", type=float, default=20.0)
    ap.add_argument("--cpu-check-steps", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--mode", choices=("full", "kernels", "traffic", "prefill", "step"), default="full")
    ap.add_argument("--summarize-pmc", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "PLAN_JSON"))
    ap.add_argument("--summarize-prefill", metavar="KERNEL_TRACE_CSV",
                    help="per-kernel table of the prefills in a rocprofv3 kernel trace of --mode prefill at --ctx")
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
                               qk_scale, P(sess.part_m), P(sess.part_l), P(sess.part_acc), st())
         for i in range(nl)],
        ["attn_split_fused_i8_kernel"])
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


def time_decode(torch, w, ctx: int, steps: int, warmup: int, extra: int):
    from lemoq.model.olmoe import DecodeSession

    sess = DecodeSession(w, [1] * ctx, max_new_tokens=warmup + 2 * steps + extra + 4)
    sess.capture()
    ttft = measure_prefill(torch, sess)
    log("ctx %d: batched prefill (TTFT) p50 %.3f ms over %d runs" % (ctx, ttft["p50"], ttft["runs"]))
    for _ in range(warmup):
        sess.graph.replay()
    torch.cuda.synchronize()
    filled0 = int(sess.filled.item())
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        sess.graph.replay()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    dev_ms = e0.elapsed_time(e1)
    # Per-step latency distribution: a second pass with an event between replays.
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    evs[0].record()
    for i in range(steps):
        sess.graph.replay()
        evs[i + 1].record()
    torch.cuda.synchronize()
    per = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(steps))
    p50, p99 = per[len(per) // 2], per[min(len(per) - 1, int(round(0.99 * (len(per) - 1))))]
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
        "ttft": ttft,
    }
    log("ctx %d: %.4f ms/token wall, %.4f device, %d steps; per-step p50 %.4f p99 %.4f ms"
        % (ctx, res["ms_per_token"], res["device_ms_per_token"], steps, p50, p99))
    return sess, res


def cpu_baseline(torch, w, cap, gpu_tokens, gpu_logits, budget_s: float, max_steps: int, snap) -> dict:
    """The CPU oracle (torch, this host's cores) decoding from the GPU's KV snapshot,
    teacher-forced on the GPU's tokens so every step compares the same input."""
    from oracle.olmoe import OracleDecoder

    kv, token, pos = snap
    t = time.time()
    host = w.to_host()
    od = OracleDecoder(host, cap.max_seq, kv=kv)
    log("cpu oracle ready in %.1fs (%d threads)" % (time.time() - t, torch.get_num_threads()))
    seq = [token] + list(gpu_tokens)
    times, agree, flips, max_kl, max_diff = [], 0, [], 0.0, 0.0
    n = 0
    for i in range(min(max_steps, len(gpu_logits))):
        t = time.perf_counter()
        lg = od.step(seq[i], pos + i)
        times.append(time.perf_counter() - t)
        ref, got = lg.double(), gpu_logits[i].double()
        p, q = torch.log_softmax(ref, -1), torch.log_softmax(got, -1)
        kl = float((p.exp() * (p - q)).sum())
        diff = float((ref - got).abs().max())
        top = torch.topk(ref, 2).values
        margin = float(top[0] - top[1])
        if int(torch.argmax(ref)) == int(torch.argmax(got)):
            agree += 1
        else:
            flips.append({"step": i, "margin": margin, "logit_diff": diff})
        max_kl, max_diff = max(max_kl, kl), max(max_diff, diff)
        n += 1
        if sum(times) > budget_s:
            break
    timed = times[1:] if len(times) > 1 else times  # first step warms the allocator
    ms = 1e3 * sum(timed) / len(timed)
    # One thread: two more steps (the second timed), the same oracle state.
    threads = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        od.step(seq[n], pos + n)
        t = time.perf_counter()
        od.step(seq[n + 1] if n + 1 < len(seq) else seq[n], pos + n + 1)
        ms_1t = 1e3 * (time.perf_counter() - t)
    finally:
        torch.set_num_threads(threads)
    log("cpu oracle: %.1f ms/token on %d threads, %.1f ms/token on 1 thread" % (ms, threads, ms_1t))
    return {
        "value": ms,
        "unit": "ms/token",
        "cores": int(threads),
        "value_1thread": ms_1t,
        "cpu_model": _cpu_model(),
        "kind": "port",
        "sample": "%d decode steps of the full OLMoE-1B-7B-shaped w8a16+KV-INT8 model by the torch-CPU oracle "
                  "from the GPU's KV snapshot at position %d, fed the GPU's greedy tokens (first step untimed)"
                  % (n, pos),
        "host_cpu_count": os.cpu_count(),
        "parity": {"steps": n, "argmax_agree": agree, "near_tie_flips": flips, "max_kl": max_kl,
                   "max_logit_diff": max_diff},
    }


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
# BASELINE attention configs as isolated kernels (fp16 and KV-INT8 split-KV)
# ---------------------------------------------------------------------------
def attention_configs(torch, hip, flusher, reps: int) -> dict:
    """Split-KV decode attention at the BASELINE shapes, cold, 16 layers' worth of
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
        r = time_cold(torch, flusher, fns, reps)
        name = "attn_%s ctx %d (split + merge, %d splits)" % (kind, ctx, ns)
        r["bytes"] = int(nbytes)
        r["gbs"] = nbytes / (r["avg_us"] * 1e-6) / 1e9
        out[name] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()}
        log("config %-44s %8.2f us avg  %7.1f GB/s" % (name, r["avg_us"], r["gbs"]))
        del caches, fns
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

        sess = DecodeSession(w, [1] * args.ctx, max_new_tokens=2)
        synthetic_cache(torch, sess, sess.ctx + 1)
        cal = copy_calibration(torch, _hip, flusher)
        kt = kernel_table(torch, _hip, w, sess, flusher, args.kernel_reps, floors=False)
        print(json.dumps({"mode": "traffic", "ctx": args.ctx, "calibration": cal, "kernels": kt}))
        return 0

    if args.mode == "step":
        from lemoq.model.olmoe import DecodeSession

        sess = DecodeSession(w, [1] * args.ctx, max_new_tokens=args.warmup + args.steps + 1)
        sess.capture()
        sess.prefill()
        sess.replay(args.warmup)
        t0 = time.perf_counter()
        sess.replay(args.steps)
        ms = (time.perf_counter() - t0) * 1e3 / args.steps
        log("ctx %d: %d replays, %.4f ms/token" % (args.ctx, args.steps, ms))
        print(json.dumps({"mode": "step", "ctx": args.ctx, "steps": args.steps, "ms_per_token": ms}))
        return 0

    if args.mode == "prefill":
        from lemoq.model.olmoe import DecodeSession

        res = {"mode": "prefill"}
        for ctx in [c for c in (args.ctx, args.ctx2) if c]:
            sess = DecodeSession(w, [1] * ctx, max_new_tokens=2)
            sess.capture()
            res["ctx%d" % ctx] = measure_prefill(torch, sess)
            log("ctx %d: TTFT p50 %.3f ms" % (ctx, res["ctx%d" % ctx]["p50"]))
            del sess
        print(json.dumps(res))
        return 0

    if args.mode == "kernels":
        from lemoq.model.olmoe import DecodeSession

        sess = DecodeSession(w, [1] * args.ctx, max_new_tokens=2)
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
    cap = _Cap(sess.max_seq)
    del sess
    r2 = None
    if args.ctx2:
        s2, r2 = time_decode(torch, w, args.ctx2, args.steps, args.warmup, 0)
        del s2
    torch.cuda.synchronize()

    cpu = None
    if check_n:
        cpu = cpu_baseline(torch, w, cap, check_tokens, check_logits, args.cpu_budget_s, check_n, snap)

    dom_name = "moe_gate_up_w8_routed"
    dom = kt[dom_name]
    traffic = _traffic_from_profiles(dom_name)
    line = {
        "metric": METRIC,
        "value": r1["ms_per_token"],
        "unit": "ms/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r1["ms_per_token"],
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
        "tokens_per_s": r1["tokens_per_s"],
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
        },
        "kernels": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()
                        if kk != "dispatch_kernels"} for k, v in kt.items()},
    }
    line["attention_configs"] = cfg
    line["step_ms_p50"], line["step_ms_p99"] = r1["step_ms_p50"], r1["step_ms_p99"]
    line["prefill"] = _prefill_summary(r1, r2)
    if r2 is not None:
        line["ctx2"] = r2
        line["ms_per_token_ctx%d" % args.ctx2] = r2["ms_per_token"]
        line["step_hbm_frac_of_peak_ctx%d" % args.ctx2] = (
            r2["step_bytes"] / (r2["device_ms_per_token"] * 1e-3) / 1e9 / HBM_PEAK_GBS)
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line))
    sys.stdout.flush()
    return 0


# Launch order of one batched prefill (lemoq.model.prefill.prefill_prompt):
# gather, layer 0's input norm, 16 x [11 launches] (each layer's combine but the
# last also writes the next layer's input norm), final norm, lm_head GEMM, then
# the greedy pick; each role with the kernel-name fragment its dispatch must carry.
PREFILL_HEAD_ROLES = (("gather_rows", "gather_rows_kernel"), ("rmsnorm (input, layer 0)", "rmsnorm_kernel"))
PREFILL_LAYER_ROLES = (("gemm_w8 qkv", "gemm_kernel<true"),
                       ("qk_rows (q/k norm, RoPE, KV-INT8)", "qk_rows_kernel"), ("attn_prefill", "attn_prefill_kernel"),
                       ("gemm_w8 o_proj (+residual)", "gemm_kernel<true"), ("rmsnorm (post-attention)", "rmsnorm_kernel"),
                       ("gemm_f16 router (split-K partials)", "gemm_kernel<false"),
                       ("route_topk (+ split-K sum)", "route_topk_kernel"),
                       ("moe_prefill_sort", "moe_sort_kernel"), ("moe_prefill_gate_up", "moe_gate_up_kernel"),
                       ("moe_prefill_down", "moe_down_kernel"))
PREFILL_COMBINE_NORM = ("moe_prefill_combine (+residual, next input norm)", "moe_combine_kernel<true")
PREFILL_COMBINE_LAST = ("moe_prefill_combine (+residual)", "moe_combine_kernel<false")
PREFILL_TAIL_ROLES = (("rmsnorm (final)", "rmsnorm_kernel"), ("gemm_w8 lm_head (last row)", "gemm_kernel<true"),
                      ("argmax_advance", "argmax_advance_kernel"))


def prefill_roles(n_layers: int = 16) -> list:
    roles = list(PREFILL_HEAD_ROLES)
    for li in range(n_layers):
        roles += list(PREFILL_LAYER_ROLES)
        roles.append(PREFILL_COMBINE_NORM if li + 1 < n_layers else PREFILL_COMBINE_LAST)
    return roles + list(PREFILL_TAIL_ROLES)


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
        "gemm_w8 lm_head (last row)": 2.0 * V * H,
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
            "e2e_32_ms": ttft + 32 * r["ms_per_token"],
            "e2e_128_ms": ttft + 128 * r["ms_per_token"],
            "reference_rtx5090_ttft_ms": REFERENCE_RTX5090_TTFT_MS.get(c),
            "reference_rtx5090_e2e_32_ms": REFERENCE_RTX5090_E2E32_MS.get(c),
        }
    return out


class _Cap:
    """Stand-in carrying the cache capacity the CPU oracle needs."""

    def __init__(self, max_seq: int) -> None:
        self.max_seq = max_seq


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
