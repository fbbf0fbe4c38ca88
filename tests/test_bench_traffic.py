"""bench.py's counter summary (CPU): two synthetic rocprofv3 counter_collection
files with known per-dispatch KiB must give back the bytes they were built
from, scaled by the calibration copy, and a dispatch order that does not follow
the plan must be rejected."""

from __future__ import annotations

import csv
import json

import pytest

import bench

COLS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
        "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
        "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]

PLAN = {
    "mode": "traffic", "ctx": 64,
    "calibration": {"copy_bytes": 1 << 20, "copies": 2, "flush_bytes": 4 << 20},
    "kernels": {
        "a": {"bytes": 1000, "launches": 2, "dispatch_kernels": ["moe_gate_up_kernel"]},
        "b": {"bytes": 500, "launches": 2, "dispatch_kernels": ["gemv_w8_kernel", "argmax_advance_kernel"]},
    },
}


def _write(path, counter, seq):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=COLS)
        w.writeheader()
        for i, (name, kib) in enumerate(seq):
            row = {c: 0 for c in COLS}
            row.update({"Dispatch_Id": i + 1, "Kernel_Name": "void (anonymous namespace)::%s<1>(Args)" % name,
                        "Counter_Name": counter, "Counter_Value": kib})
            w.writerow(row)


def _seq(copy_kib, a_kib, b_kib, c_kib):
    seq = [("rtn_w8_kernel", 99.0), ("read_probe_kernel", 4096.0), ("copy_probe_kernel", copy_kib),
           ("read_probe_kernel", 4096.0), ("copy_probe_kernel", copy_kib), ("__amd_rocclr_copyBuffer", 7.0)]
    for _ in range(2):  # one flush, then the launches of one pass
        seq.append(("read_probe_kernel", 4096.0))
        seq.append(("moe_gate_up_kernel", a_kib))
    for _ in range(2):
        seq.append(("read_probe_kernel", 4096.0))
        seq += [("gemv_w8_kernel", b_kib), ("argmax_advance_kernel", c_kib)]
    return seq


def test_summary_recovers_calibrated_bytes(tmp_path):
    # fetch counter reads 2x the true bytes (factor 0.5), write counter 1x
    _write(tmp_path / "f.csv", "FETCH_SIZE", _seq(2048.0, 8.0, 4.0, 1.0))
    _write(tmp_path / "w.csv", "WRITE_SIZE", _seq(1024.0, 1.0, 0.5, 0.25))
    (tmp_path / "plan.json").write_text("progress line\n" + json.dumps(PLAN) + "\n")
    r = bench.summarize_pmc(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), str(tmp_path / "plan.json"),
                            str(tmp_path / "out"))
    d = json.loads((tmp_path / "out" / "traffic.json").read_text())
    assert d["calibration"]["fetch_factor"] == pytest.approx(0.5)
    assert d["calibration"]["write_factor"] == pytest.approx(1.0)
    assert d["a"]["read_bytes"] == 4096 and d["a"]["write_bytes"] == 1024 and d["a"]["traffic_bytes"] == 5120
    assert d["b"]["read_bytes"] == 2560 and d["b"]["write_bytes"] == 768
    assert d["b"]["algorithmic_bytes"] == 500 and "| b | 500 |" in r["table"]


def test_summary_rejects_dispatches_out_of_plan(tmp_path):
    seq = _seq(1024.0, 1.0, 1.0, 1.0)
    seq[7] = ("gemv_w8_kernel", 1.0)  # the plan expects moe_gate_up_kernel there
    seq.insert(3, ("__amd_rocclr_copyBuffer", 5.0))  # not a plan kernel: skipped
    _write(tmp_path / "f.csv", "FETCH_SIZE", seq)
    _write(tmp_path / "w.csv", "WRITE_SIZE", _seq(1024.0, 1.0, 1.0, 1.0))
    (tmp_path / "plan.json").write_text(json.dumps(PLAN))
    with pytest.raises(SystemExit, match="gemv_w8_kernel.*expects moe_gate_up_kernel"):
        bench.summarize_pmc(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), str(tmp_path / "plan.json"),
                            str(tmp_path / "out"))


def test_in_graph_duration_read_from_trace_table(tmp_path, monkeypatch):
    """roofline.in_graph_avg_us comes from the committed kernel-trace table: the
    row of the dispatch name, its in-graph column; absent rows or files give None."""
    prof = tmp_path / "profiles"
    prof.mkdir()
    (prof / "bench_kernel_trace.md").write_text(
        "# trace\n\n| kernel | in-graph / other launches | avg us | isolated cold launches | avg us |\n"
        "|---|---|---|---|---|\n"
        "| moe_gate_up_kernel<4> | 288 | 242.14 | 0 | - |\n"
        "| moe_gate_up_kernel<2, 2, 1, true> | 2720 | 8.30 | 64 | 7.96 |\n"
        "| attn_split_kernel<128, true> | 0 | - | 128 | 11.84 |\n")
    monkeypatch.setattr(bench, "REPO", str(tmp_path))
    assert bench._in_graph_from_profiles("moe_gate_up_kernel<2, 2, 1, true>") == 8.30
    assert bench._in_graph_from_profiles("attn_split_kernel<128, true>") is None   # no in-graph launches
    assert bench._in_graph_from_profiles("moe_down_kernel<1, 4, true>") is None
    monkeypatch.setattr(bench, "REPO", str(tmp_path / "missing"))
    assert bench._in_graph_from_profiles("moe_gate_up_kernel<2, 2, 1, true>") is None


def test_summarize_step_timeline(tmp_path):
    """bench.py --summarize-step on a synthetic kernel trace of two whole decode
    steps (16 layers x 6 launches + lm_head + argmax, each kernel 2 us with a
    1 us gap) plus a prefill seed pick (argmax alone): two steps, span and busy
    time of each, per-kernel averages."""
    path = tmp_path / "trace.csv"
    names = [k for _, k in bench.STEP_LAYER_KERNELS] * 16 + [k for _, k in bench.STEP_TAIL_KERNELS]
    names = [k + ", false>" if k.endswith("<true") else k for k in names]  # the kernel's full instance name
    rows, t = [], 1000
    rows.append(("void (anonymous namespace)::argmax_advance_kernel<true, false>(args)", t, t + 2000))  # seed pick
    t += 5000
    for _ in range(2):
        for n in names:
            rows.append(("void (anonymous namespace)::%s(args)" % n.replace("<", "<").strip(), t, t + 2000))
            t += 3000
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for n, a, b in rows:
            w.writerow({"Kernel_Name": n, "Start_Timestamp": a, "End_Timestamp": b})
    out = bench.summarize_step(str(path))
    per_step = 16 * 6 + 2
    assert out.startswith("2 whole steps of %d launches" % per_step)
    span = (per_step - 1) * 3.0 + 2.0
    assert "step span p50 %.1f us" % span in out
    assert "kernel busy time p50 %.1f us" % (per_step * 2.0) in out
    assert "| qkv (+ input RMSNorm) | 16 | 2.00 |" in out
    assert "| argmax + advance | 1 | 2.00 |" in out


def test_summarize_step_timeline_of_the_4bit_step(tmp_path):
    """The 4-bit step (bench.py --mode step --weights w4a16): 98 launches told
    apart by position, the trace recognised by the fp16 lm_head kernel; the prompt's steps
    come first and --summarize-last keeps the decode steps.  Synthetic trace: 3 prompt steps (1 us kernels) and 2 decode
    steps (role i lasts i + 1 us), 1 us gaps."""
    path = tmp_path / "trace_w4.csv"
    layer = ["gemv_q_kernel<2, 1, 2, false, true>", "attn_split_fused_i8_kernel<128, 4, 3>",
             "merge_oproj_q4_kernel<16>", "router_resid_kernel<2, 4>",
             "moe_gate_up_q4_kernel<1, 2, 16, 1>", "moe_down_q4_kernel<1, 4, 8>"]
    step = layer * 16 + ["lm_head_f16_argmax_kernel<2, true>", "argmax_advance_kernel<true, false>"]
    rows, t = [("void at::native::fill_kernel(args)", 0, 500)], 1000
    for s in range(5):
        for i, n in enumerate(step):
            d = 1000 if s < 3 else 1000 * (1 + (i % 6 if i < 96 else 6 + (i - 96)))
            rows.append(("void (anonymous namespace)::%s(args)" % n, t, t + d))
            t += d + 1000
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for n, a, b in rows:
            w.writerow({"Kernel_Name": n, "Start_Timestamp": a, "End_Timestamp": b})
    out = bench.summarize_step(str(path), last=2)
    assert out.startswith("2 whole steps of 98 launches"), out
    assert "| qkv (4-bit, + input RMSNorm) | 16 | 1.00 |" in out
    assert "| merge + o_proj (4-bit) | 16 | 3.00 |" in out
    assert "| residual + norm + router | 16 | 4.00 |" in out
    assert "| lm_head fp16 (+ final norm, argmax partials) | 1 | 7.00 |" in out
    assert "| argmax + advance | 1 | 8.00 |" in out
    assert bench.summarize_step(str(path)).startswith("5 whole steps of 98 launches")
