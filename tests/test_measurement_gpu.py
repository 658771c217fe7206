"""bench.py's output contract on a GPU: one JSON line on stdout with the
metric, whole-job value, roofline, CPU-baseline and raw-transfer objects,
run briefly (2 timed + 2 recorded steps per pass) as a child process."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_prints_one_contract_line(device):
    cmd = [sys.executable, "-u", os.path.join(ROOT, "bench.py"), "--steps", "2", "--warmup", "1",
           "--prewarm", "2", "--cpu-seconds", "0.5", "--resident-reps", "2",
           "--config-steps", "2", "--layers", "2", "--context", "64", "--tree-nodes", "8",
           "--expert-sets", "2"]
    print("bench contract run:", " ".join(cmd[2:]), flush=True)
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=170, cwd=ROOT)
    assert out.returncode == 0, out.stderr[-3000:]
    lines = [line for line in out.stdout.splitlines() if line.strip()]
    assert len(lines) == 1, out.stdout[-2000:]
    d = json.loads(lines[0])
    assert d["metric"].startswith("verified tree tokens/s per MoE layer")
    assert d["unit"] == "tokens/s" and d["value"] > 0 and d["n_gpus"] == 1
    assert d["steps"] == 2 and d["warmup"] == 1 and d["higher_is_better"] is True
    assert d["value"] == pytest.approx(2 * 64 / (d["ms_per_step"] * 2e-3), rel=1e-6)
    assert d["vs_baseline"] is None and d["dtype"] == "bf16" and d["data"].startswith("synthetic")
    assert "64 tree tokens" in d["config"]["workload"]
    r = d["roofline"]
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert 0 < r["achieved"] < r["peak"] and r["frac"] == pytest.approx(r["achieved"] / r["peak"])
    assert r["traffic"] is None or r["traffic"] > 0
    c = d["cpu_baseline"]
    assert c["kind"] == "port" and c["value"] > 0 and c["cores"] >= 1 and c["sample"]
    assert d["device_ms_per_step"]["n"] == 2
    assert d["h2d"]["link_peak_gbs"] > 0 and 0 <= d["overlap"] <= 1
    # coded transfers by default: ~67% of the expert bytes over the link
    h = d["h2d"]
    assert d["config"]["transfer"] == h["transfer"] == "coded"
    assert 0.64 * h["expert_bytes"] < h["bytes"] < 0.69 * h["expert_bytes"]
    dec = d["decode"]
    assert dec["count"] == h["transfers"] and 0 < dec["frac"] < 1
    # the reference's raw transfers, measured beside the coded headline
    raw = d["raw_transfer"]
    assert raw["value"] > 0 and raw["unit"] == "tokens/s"
    assert raw["value"] == pytest.approx(2 * 64 / (raw["ms_per_step"] * 2e-3), rel=1e-6)
    assert raw["misses_per_step"] > 0 and raw["h2d_gbs"] > 0
    assert 0 < raw["k3_in_step_gbs"] < 8000.0
    # the other configurations, each in a short run of its own
    other = d["other_configs"]
    assert set(other) == {"resident16", "sweep", "verify48", "cold48", "verify48_ready_demand",
                          "cold48_ready_demand"}
    assert all("error" not in v for v in other.values()), other
    assert other["resident16"]["value"] > 0 and 0 < other["resident16"]["k3_frac"] < 1
    assert [p["tokens"] for p in other["sweep"]["points"]] == [1, 8, 32, 64, 128]
    assert all(p["tokens_per_s"] > 0 for p in other["sweep"]["points"])
    for name in ("verify48", "cold48", "verify48_ready_demand", "cold48_ready_demand"):
        assert other[name]["value"] > 0 and "2 layers" in other[name]["workload"]
        assert other[name]["executor"] == ("ready_demand" if "ready" in name else "layer")



@pytest.mark.parametrize("workload,executor", [("cold48", "predicted"), ("verify48", "ready_demand")])
def test_bench_48_layer_forward_under_the_prefetch_scheduler(device, workload, executor):
    """The 48-layer workloads under the reference's executor, shrunk to 2
    layers, an 8-node tree and a 64-token context: one contract line whose
    scheduler statistics show complete forwards (and, with predictions,
    every routed expert predicted)."""
    cmd = [sys.executable, "-u", os.path.join(ROOT, "bench.py"), "--workload", workload,
           "--executor", executor, "--layers", "2", "--tree-nodes", "8", "--context", "64",
           "--steps", "2", "--warmup", "1", "--record", "none"]
    print("bench scheduler run:", " ".join(cmd[2:]), flush=True)
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=110, cwd=ROOT)
    assert out.returncode == 0, out.stderr[-3000:]
    lines = [line for line in out.stdout.splitlines() if line.strip()]
    assert len(lines) == 1, out.stdout[-2000:]
    d = json.loads(lines[0])
    assert d["value"] > 0 and d["config"]["executor"] == executor and d["config"]["layers"] == 2
    assert "2 distinct expert sets" in d["data"]
    assert d["config"]["transfer"] == d["h2d"]["transfer"] == "coded"
    s = d["scheduler"]
    assert s["complete"] and 1 <= s["peak_inflight"] <= s["max_inflight"] == 2
    per = s["per_forward"]
    assert per["actual_experts"] > 0
    if executor == "predicted":
        assert per["predicted_experts"] == per["actual_experts"]
        assert per["unused_prediction_copies"] == 0
    else:
        assert per["predicted_experts"] == 0 and per["prediction_copies"] == 0


def test_bench_link_breakdown_of_the_48_layer_forward(device):
    """--record copies on the cold forward, shrunk to 2 layers: the link
    block counts every copy of the recorded pass and one boundary per
    forward, and its times add up."""
    cmd = [sys.executable, "-u", os.path.join(ROOT, "bench.py"), "--workload", "cold48",
           "--layers", "2", "--tree-nodes", "8", "--context", "64", "--expert-sets", "2",
           "--steps", "2", "--warmup", "1", "--record", "copies", "--cpu-seconds", "0"]
    print("bench link run:", " ".join(cmd[2:]), flush=True)
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=110, cwd=ROOT)
    assert out.returncode == 0, out.stderr[-3000:]
    d = json.loads([line for line in out.stdout.splitlines() if line.strip()][-1])
    link = d["link"]
    assert link["forwards"] == 2
    assert link["copies"] == d["h2d"]["transfers"] > 0
    assert link["boundary_idle_us"]["boundaries"] == 2  # layer 1's router, per forward
    ms = link["ms_per_forward"]
    assert all(v >= 0 for v in ms.values()) and ms["busy"] > 0
    assert ms["busy"] == pytest.approx(ms["one"] + ms["two"], rel=1e-6)
    device_ms = d["device_ms_per_step"]["median"]
    spent = ms["busy"] + ms["boundary"] + ms["within"] + ms["prologue"] + ms["epilogue"]
    assert spent == pytest.approx(device_ms, rel=0.5)
