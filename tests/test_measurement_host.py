"""CPU checks of the measurement code: the rocprofv3 summaries of
specfit_amd/pmc.py on synthetic counter and trace files, and the bench
helpers (copy/K3 interval union, per-step statistics, the committed traffic
ratio, per-workload step defaults)."""
import csv
import os
import subprocess
import sys

import pytest

import bench
from specfit_amd import pmc

H, I = pmc.HIDDEN, pmc.INTERMEDIATE
GATEUP_BYTES = 2 * I * H * 2     # gate + up rows of one expert
DOWN_BYTES = H * I * 2


def _name(kind: str, nt: int, mc: int = 2) -> str:
    nb = 8 if kind == "gateup" else 3
    return (f"void (anonymous namespace)::{kind}_mfma_kernel<((anonymous namespace)::Resolve)0, "
            f"{mc}, {nb}, {nt}>((anonymous namespace)::SwigluArgs)")


def _grid(kind: str, nt: int, experts: int) -> int:
    tiles = I // (8 * nt) if kind == "gateup" else H // (16 * nt)
    return experts * tiles * pmc.THREADS


def test_tile_width_and_weight_bytes_from_kernel_names():
    for nt in (1, 2):
        for n in (1, 3, 45):
            assert pmc._k3_weight_bytes(_name("gateup", nt), _grid("gateup", nt, n)) == n * GATEUP_BYTES
            assert pmc._k3_weight_bytes(_name("down", nt), _grid("down", nt, n)) == n * DOWN_BYTES
    assert pmc._tile_width(_name("down", 1)) == 1
    assert pmc._k3_weight_bytes("void combine_kernel<true>(...)", 1024) is None
    with pytest.raises(ValueError):
        pmc._tile_width("gateup_mfma_kernel(no template)")


CAL = "void at::native::vectorized_elementwise_kernel<4, at::native::neg_kernel_cuda(...)>"


def _counter_dir(tmp_path, name, counter, rows):
    d = tmp_path / name
    d.mkdir()
    with open(d / "k3_counter_collection.csv", "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"])
        for i, (kname, grid, kib) in enumerate(rows):
            # two partial rows per dispatch (the summary adds them)
            w.writerow([i, kname, grid, counter, kib / 2])
            w.writerow([i, kname, grid, counter, kib / 2])
    return str(d)


def test_traffic_summary_calibrates_and_splits_phases(tmp_path):
    # FETCH counts half the bytes (scale 2), WRITE counts all (scale 1).
    cal_kib = (256 << 20) / 1024
    launches_in = [(2, 3), (1, 5)]   # (tile width, experts) of the in-step launches
    fetch, write = [], []
    for nt, n in launches_in:
        for kind, wb in (("gateup", GATEUP_BYTES), ("down", DOWN_BYTES)):
            fetch.append((_name(kind, nt), _grid(kind, nt, n), n * wb * 1.05 / 1024 / 2))
            write.append((_name(kind, nt), _grid(kind, nt, n), n * wb * 0.01 / 1024))
    # two decodes of coded records: 1152 chunks of 4096 values, 6.3 MB read,
    # every value written once
    dec = "void (anonymous namespace)::decode_kernel((anonymous namespace)::DecodeArgs)"
    values = 1152 * 4096
    for _ in range(2):
        fetch.append((dec, 1152 * pmc.THREADS, 6.3e6 / 1024 / 2))
        write.append((dec, 1152 * pmc.THREADS, 2 * values / 1024))
    fetch.append((CAL, 1 << 20, cal_kib / 2))
    write.append((CAL, 1 << 20, cal_kib))
    for kind, wb in (("gateup", GATEUP_BYTES), ("down", DOWN_BYTES)):  # all-resident, 45 experts
        fetch.append((_name(kind, 2), _grid(kind, 2, 45), 45 * wb * 1.02 / 1024 / 2))
        write.append((_name(kind, 2), _grid(kind, 2, 45), 0.0))
    text = pmc.summarize(_counter_dir(tmp_path, "fetch", "FETCH_SIZE", fetch),
                         _counter_dir(tmp_path, "write", "WRITE_SIZE", write), command="cmd")
    ratios = {line.split(":")[0]: float(line.split(":")[1]) for line in text.splitlines()
              if line.startswith("traffic_ratio_")}
    assert ratios["traffic_ratio_in_step"] == pytest.approx(1.06, abs=1e-6)
    assert ratios["traffic_ratio_all_resident"] == pytest.approx(1.02, abs=1e-6)
    assert "| FETCH_SIZE |" in text and "2.0000" in text and "    cmd" in text
    dec_bytes = {line.split(":")[0]: float(line.split(":")[1]) for line in text.splitlines()
                 if line.startswith("decode_")}
    assert dec_bytes["decode_fetch_bytes"] == pytest.approx(6.3e6, rel=1e-9)
    assert dec_bytes["decode_write_bytes"] == pytest.approx(2 * values, rel=1e-9)
    assert "| 2 | 6.300 | 9.437 | 9.437 | 1.000 |" in text


def test_traffic_summary_rejects_mismatched_runs(tmp_path):
    row = (_name("gateup", 2), _grid("gateup", 2, 1), 100.0)
    other = (_name("down", 2), _grid("down", 2, 1), 100.0)
    cal = (CAL, 1 << 20, 1000.0)
    f = _counter_dir(tmp_path, "f", "FETCH_SIZE", [row, other, cal])
    w = _counter_dir(tmp_path, "w", "WRITE_SIZE", [other, row, cal])
    with pytest.raises(RuntimeError, match="different K3 dispatch sequences"):
        pmc.summarize(f, w)
    nocal = _counter_dir(tmp_path, "n", "FETCH_SIZE", [row, other])
    with pytest.raises(RuntimeError, match="calibration"):
        pmc.summarize(nocal, w)


def test_trace_summary_averages_k3_launches_per_phase(tmp_path):
    d = tmp_path / "trace"
    d.mkdir()
    rows, t = [], 0
    def add(name, grid, dur_ns):
        nonlocal t
        rows.append({"Kernel_Name": name, "Grid_Size_X": grid, "Start_Timestamp": t,
                     "End_Timestamp": t + dur_ns})
        t += dur_ns + 1000
    for _ in range(3):  # in-step: 2 experts, narrow, gate/up 10 us + down 6 us
        add(_name("gateup", 1, 0), _grid("gateup", 1, 2), 10_000)
        add(_name("down", 1, 0), _grid("down", 1, 2), 6_000)
    add(CAL, 1 << 20, 90_000)
    add(_name("gateup", 2), _grid("gateup", 2, 45), 55_000)
    add(_name("down", 2), _grid("down", 2, 45), 33_000)
    table = lambda n: n.replace("Resolve)0", "Resolve)1")  # slot-table launch over 128 entries
    add(table(_name("gateup", 2, 0)), _grid("gateup", 2, 128), 80_000)
    add(table(_name("down", 2, 0)), _grid("down", 2, 128), 40_000)
    with open(d / "k3_kernel_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    with open(d / "k3_kernel_stats.csv", "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["Name", "Calls", "AverageNs", "MinNs", "MaxNs", "Percentage"])
        w.writerow([_name("gateup", 2), 1, 55000, 55000, 55000, 40.0])
        w.writerow(["void at::native::elementwise_kernel<128>(int)", 9, 2000, 1000, 3000, 1.0])
        w.writerow(["void (anonymous namespace)::qk_norm_rope_kernel(unsigned short const*)", 48,
                    4900, 4500, 5200, 2.0])
    text = pmc.summarize_trace(str(d))
    library = text.split("## Kernels of libspecfit_amd")[1].split("##")[0]
    assert "`qk_norm_rope_kernel` | 48 | 4.90 | 4.50 | 5.20 | 2.0% |" in library
    assert "gateup_mfma_kernel" in library and "elementwise_kernel" not in library
    lines = {l.split("|")[1].strip(): l for l in text.splitlines()
             if l.startswith("| in-step") or l.startswith("| all-resident")}
    table_row = [c.strip() for c in lines["all-resident, slot table"].split("|")[1:-1]]
    assert table_row[1:] == ["1", "80.00", "40.00", "120.00", "n/a", "n/a"]
    in_step = [c.strip() for c in lines["in-step"].split("|")[1:-1]]
    assert in_step[1:5] == ["3", "10.00", "6.00", "16.00"]
    assert float(in_step[5]) == pytest.approx(2 * (GATEUP_BYTES + DOWN_BYTES) / 1e6, abs=0.01)
    resident = [c.strip() for c in lines["all-resident"].split("|")[1:-1]]
    assert resident[1:5] == ["1", "55.00", "33.00", "88.00"]
    assert "`gateup_mfma_kernel<(Resolve)0, 2, 8, 2>`" in text


class _Ev:
    def __init__(self, t):
        self.t = t

    def elapsed_time(self, other):
        return other.t - self.t


def test_trace_summary_without_split_starts_at_the_first_router(tmp_path):
    d = tmp_path / "trace"
    d.mkdir()
    rows, t = [], 0
    for name, dur in (("void encode_setup_kernel(int)", 50_000),
                      ("void (anonymous namespace)::router_logits_kernel<4>(int)", 6_000),
                      ("void (anonymous namespace)::decode_kernel(int)", 10_000),
                      ("void (anonymous namespace)::decode_kernel(int)", 12_000),
                      ("void (anonymous namespace)::router_logits_kernel<4>(int)", 4_000)):
        rows.append({"Kernel_Name": name, "Grid_Size_X": 1, "Start_Timestamp": t,
                     "End_Timestamp": t + dur})
        t += dur + 500
    with open(d / "f_kernel_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    with open(d / "f_kernel_stats.csv", "w", newline="") as fh:
        csv.writer(fh).writerow(["Name", "Calls", "AverageNs", "MinNs", "MaxNs", "Percentage"])
    text = pmc.summarize_trace(str(d), split=False)
    assert "from the first router launch on" in text and "encode_setup_kernel" not in text
    assert "| `decode_kernel` | 2 | 11.00 | 10.00 | 12.00 | 68.8% |" in text
    assert "| `router_logits_kernel<4>` | 2 | 5.00 | 4.00 | 6.00 | 31.2% |" in text


def test_bench_helpers():
    assert bench._union_length([(0, 2), (1, 3), (5, 6)]) == 4
    assert bench._union_length([]) == 0
    assert bench.step_stats([]) is None
    st = bench.step_stats([(_Ev(0), _Ev(x)) for x in (5.0, 1.0, 3.0, 2.0, 4.0)])
    assert st == {"median": 3.0, "p10": 1.0, "p90": 5.0, "n": 5}
    ratio, source = bench._traffic_ratio()
    assert 1.0 <= ratio < 1.2 and source.startswith("profiles/k3_traffic")


def test_decode_stats():
    class _Rec:
        decodes = []

    assert bench.decode_stats(_Rec()) is None
    rec = _Rec()
    # two decodes of a 100-byte record of 40 values, 0.002 and 0.004 ms
    rec.decodes = [(100, 40, _Ev(0.0), _Ev(0.002)), (100, 40, _Ev(1.0), _Ev(1.004))]
    d = bench.decode_stats(rec)
    assert d["count"] == 2 and d["alg_bytes_per_decode"] == 180
    assert d["avg_us"] == pytest.approx(3.0)
    assert d["gbs"] == pytest.approx(360 / 6e-6 / 1e9)
    assert d["frac"] == pytest.approx(d["gbs"] / bench.HBM_PEAK_GBS)


def test_link_stats_splits_idle_link_time():
    class _Rec:
        copy_spans, marks = [], []

    assert bench.link_stats(_Rec(), []) is None
    rec = _Rec()
    ms = lambda *xs: [_Ev(x) for x in xs]
    # Forward 1 (0 .. 1 ms): two overlapping copies, a 50 us gap inside
    # layer 0, a 150 us gap across layer 1's router (0.5 ms), one more copy.
    # Forward 2 (2 .. 3 ms): copies run through layer 1's router.
    rec.copy_spans = [tuple(ms(a, b)) for a, b in
                      ((0.05, 0.2), (0.1, 0.3), (0.35, 0.45), (0.6, 0.9), (2.1, 2.6),
                       (2.55, 2.9))]
    rec.marks = [(0, _Ev(0.0)), (1, _Ev(0.5)), (0, _Ev(2.0)), (1, _Ev(2.5))]
    steps = [tuple(ms(0.0, 1.0)), tuple(ms(2.0, 3.0))]
    got = bench.link_stats(rec, steps)
    assert got["forwards"] == 2 and got["copies"] == 6
    assert got["boundary_idle_us"]["boundaries"] == 2
    assert got["boundary_idle_us"]["mean"] == pytest.approx(75.0)
    assert got["boundary_idle_us"]["median"] == pytest.approx(150.0)
    want = dict(busy=0.725, one=0.65, two=0.075, boundary=0.075, within=0.025, prologue=0.075,
                epilogue=0.1)
    for key, value in want.items():
        assert got["ms_per_forward"][key] == pytest.approx(value), key


def test_link_stats_forward_without_copies_and_copies_through_every_boundary():
    """A forward whose experts were all resident (no copies) counts as a
    forward but contributes no link time; copies that run through every
    router give zero boundary idle."""
    class _Rec:
        copy_spans, marks = [], []

    rec = _Rec()
    rec.copy_spans = [(_Ev(2.1), _Ev(2.6)), (_Ev(2.5), _Ev(2.95))]
    rec.marks = [(0, _Ev(0.0)), (1, _Ev(0.5)), (0, _Ev(2.0)), (1, _Ev(2.4)), (2, _Ev(2.55))]
    steps = [(_Ev(0.0), _Ev(1.0)), (_Ev(2.0), _Ev(3.0))]
    got = bench.link_stats(rec, steps)
    assert got["forwards"] == 2 and got["copies"] == 2
    b = got["boundary_idle_us"]
    # Forward 2: layer 1's router (2.4 ms) falls before the first copy, so
    # no gap holds it; layer 2's (2.55 ms) falls inside the copies.
    assert b["boundaries"] == 2 and b["median"] == 0.0 and b["mean"] == 0.0
    ms = got["ms_per_forward"]
    assert ms["busy"] == pytest.approx(0.85 / 2)
    assert ms["two"] == pytest.approx(0.1 / 2) and ms["one"] == pytest.approx(0.75 / 2)
    assert ms["within"] == 0.0 and ms["boundary"] == 0.0
    assert ms["prologue"] == pytest.approx(0.1 / 2) and ms["epilogue"] == pytest.approx(0.05 / 2)


@pytest.mark.parametrize("argv,steps", [([], 50), (["--workload", "verify48"], 10),
                                        (["--workload", "cold48"], 10), (["--steps", "7"], 7)])
def test_bench_step_defaults(monkeypatch, argv, steps):
    monkeypatch.setattr(sys, "argv", ["bench.py", *argv])
    assert bench.parse_args().steps == steps


def test_bench_refuses_more_than_one_gpu():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=60, cwd=root)
    assert out.returncode == 2 and "one GPU only" in out.stderr and not out.stdout.strip()


@pytest.mark.parametrize("argv,ok,lookahead", [
    (["--executor", "ready_demand"], False, None),
    (["--workload", "verify48", "--executor", "predicted"], True, 1),
    (["--workload", "verify48", "--executor", "ready_demand"], True, 0),
    (["--workload", "cold48", "--executor", "predicted"], True, 1),
    (["--workload", "cold48", "--executor", "ready_demand", "--lookahead", "2"], True, 2)])
def test_bench_executor_applies_to_the_48_layer_forwards(monkeypatch, argv, ok, lookahead):
    monkeypatch.setattr(sys, "argv", ["bench.py", *argv])
    if ok:
        args = bench.parse_args()
        assert args.executor == argv[3] and args.lookahead == lookahead
    else:
        with pytest.raises(SystemExit):
            bench.parse_args()
