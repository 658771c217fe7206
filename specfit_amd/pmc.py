"""HBM traffic of the K3 dispatches from two rocprofv3 counter runs.

Usage (after two runs of the same ``bench.py`` command, one under
``rocprofv3 --pmc FETCH_SIZE`` and one under ``rocprofv3 --pmc WRITE_SIZE``,
each with ``--output-format csv``)::

    python -m specfit_amd.pmc --fetch <dir1> --write <dir2> [--command "..."]

``bench.py`` runs a plain elementwise kernel of known size between the
in-step phase and the all-resident phase (``torch.neg`` over 256 MiB of
fp32: 256 MiB read, 256 MiB written).  It calibrates each counter
(scale = known KiB / counted KiB) and splits the K3 dispatches into the
in-step ones (before it) and the all-resident ones (after it).

The summary is markdown; its ``traffic_ratio_in_step:`` line (scaled
FETCH + WRITE bytes of the in-step K3 dispatches over their algorithmic
weight bytes) is what ``bench.py`` reports as ``roofline.traffic``.
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import re
import sys
from collections import defaultdict

CALIBRATION_BYTES = 256 << 20   # read and written by the calibration kernel
CALIBRATION_TAG = "neg"         # substring of the calibration kernel's name
HIDDEN, INTERMEDIATE = 2048, 768
THREADS = 256
DECODE_CHUNK = 4096             # values per decode workgroup (SF_DECODE_CHUNK)


def _rows(run_dir: str) -> list[dict]:
    files = glob.glob(os.path.join(run_dir, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise FileNotFoundError(f"no *counter_collection.csv under {run_dir}")
    out = []
    for f in files:
        with open(f, newline="") as fh:
            out.extend(csv.DictReader(fh))
    return out


def _per_dispatch(run_dir: str, counter: str) -> list[tuple[int, str, int, float]]:
    """(dispatch id, kernel name, grid size, counter value in KiB), in dispatch order."""
    acc: dict[int, list] = {}
    for r in _rows(run_dir):
        if r.get("Counter_Name") != counter:
            continue
        d = int(r["Dispatch_Id"])
        if d not in acc:
            acc[d] = [r["Kernel_Name"], int(r["Grid_Size"]), 0.0]
        acc[d][2] += float(r["Counter_Value"])
    return [(d, *acc[d]) for d in sorted(acc)]


def _tile_width(name: str) -> int:
    """The kernel's last template argument: 1 for narrow tiles (8 gate/up
    columns, 16 down columns per workgroup), 2 for wide ones (16 / 32)."""
    m = re.search(r"_mfma_kernel<([^<>]*)>", name)
    if not m:
        raise ValueError(f"no template arguments in kernel name {name!r}")
    return int(m.group(1).split(",")[-1])


def _is_table(name: str) -> bool:
    """A slot-table K3 dispatch (Resolve 1): one workgroup set per table
    entry, whether or not that expert has rows."""
    m = re.search(r"Resolve\)(\d)", name)
    return bool(m) and m.group(1) == "1"


def _k3_weight_bytes(name: str, grid: int) -> int | None:
    if "gateup_mfma_kernel" in name:
        cols = 8 * _tile_width(name)
        return grid // (INTERMEDIATE // cols * THREADS) * 2 * INTERMEDIATE * HIDDEN * 2
    if "down_mfma_kernel" in name:
        cols = 16 * _tile_width(name)
        return grid // (HIDDEN // cols * THREADS) * HIDDEN * INTERMEDIATE * 2
    return None


def _split(disp):
    """Scale factor from the calibration kernel; K3 dispatches before/after it."""
    cal = [i for i, (_, name, _, _) in enumerate(disp) if CALIBRATION_TAG in name]
    if not cal:
        raise RuntimeError("calibration kernel not found in the counter run")
    counted = disp[cal[0]][3]
    scale = (CALIBRATION_BYTES / 1024.0) / counted
    before = [x for x in disp[:cal[0]] if _k3_weight_bytes(x[1], x[2]) is not None]
    after = [x for x in disp[cal[-1] + 1:] if _k3_weight_bytes(x[1], x[2]) is not None]
    return counted, scale, before, after


def summarize(fetch_dir: str, write_dir: str, command: str | None = None) -> str:
    f_disp = _per_dispatch(fetch_dir, "FETCH_SIZE")
    w_disp = _per_dispatch(write_dir, "WRITE_SIZE")
    f_cnt, f_scale, f_in, f_res = _split(f_disp)
    w_cnt, w_scale, w_in, w_res = _split(w_disp)

    def phase(fd, wd):
        if len(fd) != len(wd) or len(fd) % 2:
            raise RuntimeError("FETCH and WRITE runs saw different K3 dispatch sequences")
        kinds = defaultdict(lambda: [0, 0.0, 0.0, 0])
        for (_, name, grid, fk), (_, name2, grid2, wk) in zip(fd, wd):
            if name != name2 or grid != grid2:
                raise RuntimeError("FETCH and WRITE runs saw different K3 dispatch sequences")
            key = "gate/up" if "gateup" in name else "down"
            k = kinds[key]
            k[0] += 1
            k[1] += fk * 1024 * f_scale
            k[2] += wk * 1024 * w_scale
            k[3] += _k3_weight_bytes(name, grid)
        pairs = len(fd) // 2
        fetch = sum(v[1] for v in kinds.values())
        write = sum(v[2] for v in kinds.values())
        alg = sum(v[3] for v in kinds.values())
        return pairs, fetch, write, alg, dict(kinds)

    lines = ["# K3 HBM traffic (rocprofv3 FETCH_SIZE / WRITE_SIZE) — Qwen3-30B-A3B MoE layer, "
             "64 tree tokens, 24-slot cache", ""]
    if command:
        lines += ["Commands (one counter per run; run from /tmp with TMPDIR=/tmp; `<repo>` is "
                  "the repository root):", "", "    " + command.replace("\n", "\n    "), ""]
    lines += ["## Calibration (plain elementwise kernel, 256 MiB read + 256 MiB written)", "",
              "| counter | counted KiB | known KiB | scale |", "|---|---|---|---|",
              f"| FETCH_SIZE | {f_cnt:.0f} | {CALIBRATION_BYTES / 1024:.0f} | {f_scale:.4f} |",
              f"| WRITE_SIZE | {w_cnt:.0f} | {CALIBRATION_BYTES / 1024:.0f} | {w_scale:.4f} |", "",
              "## K3 dispatches (scaled bytes; algorithmic = expert weight bytes of the "
              "dispatch's experts)", "",
              "| phase | K3 launches | kernel | dispatches | fetch MB | write MB | "
              "weight MB | fetch / weight |", "|---|---|---|---|---|---|---|---|"]
    ratios = {}
    for label, fd, wd in (("in-step", f_in, w_in), ("all-resident", f_res, w_res)):
        if not fd:
            continue
        pairs, fetch, write, alg, kinds = phase(fd, wd)
        for key, (n, fb, wb, ab) in sorted(kinds.items(), reverse=True):
            lines.append(f"| {label} | {pairs} | {key} | {n} | {fb / n / 1e6:.2f} | "
                         f"{wb / n / 1e6:.3f} | {ab / n / 1e6:.2f} | {fb / ab:.3f} |")
        ratios[label] = ((fetch + write) / alg, fetch / pairs, write / pairs, alg / pairs)
    # Coded-transfer decodes (sf_expert_decode) before the calibration kernel.
    f_cal = [i for i, d in enumerate(f_disp) if CALIBRATION_TAG in d[1]][0]
    w_cal = [i for i, d in enumerate(w_disp) if CALIBRATION_TAG in d[1]][0]
    f_dec = [d for d in f_disp[:f_cal] if "decode_kernel" in d[1]]
    w_dec = [d for d in w_disp[:w_cal] if "decode_kernel" in d[1]]
    if f_dec and len(f_dec) == len(w_dec):
        fetch = sum(d[3] for d in f_dec) * 1024 * f_scale / len(f_dec)
        write = sum(d[3] for d in w_dec) * 1024 * w_scale / len(w_dec)
        values = f_dec[0][2] // THREADS * DECODE_CHUNK  # one workgroup per chunk
        lines += ["", "## Decodes of coded records (`decode_kernel`, scaled bytes per dispatch)", "",
                  "| dispatches | fetch MB | write MB | values written (bf16 MB) | "
                  "write / values |", "|---|---|---|---|---|",
                  f"| {len(f_dec)} | {fetch / 1e6:.3f} | {write / 1e6:.3f} | "
                  f"{2 * values / 1e6:.3f} | {write / (2 * values):.3f} |", "",
                  f"decode_fetch_bytes: {fetch:.0f}", f"decode_write_bytes: {write:.0f}"]
    lines.append("")
    for label, (ratio, fpl, wpl, apl) in ratios.items():
        key = label.replace("-", "_")
        lines.append(f"- {label}: per K3 launch (gate/up + down) {fpl / 1e6:.2f} MB fetched, "
                     f"{wpl / 1e6:.3f} MB written, {apl / 1e6:.2f} MB of expert weights; "
                     f"(fetch + write) / weights = {ratio:.4f}")
        lines.append(f"")
        lines.append(f"traffic_ratio_{key}: {ratio:.6f}")
        lines.append("")
    return "\n".join(lines) + "\n"


# Kernel names of libspecfit_amd (K1-K8), listed in the trace summaries.
LIBRARY_KERNELS = ("router_logits_kernel", "router_select_kernel", "dispatch_kernel",
                   "gateup_mfma_kernel", "down_mfma_kernel", "gateup_generic_kernel",
                   "down_generic_kernel", "combine_kernel", "decode_kernel",
                   "tree_attention_kernel", "tree_attention_mfma_kernel", "rms_norm_kernel",
                   "qk_norm_rope_kernel", "router_topk_scalar_kernel")


FORWARD_START = "router_logits_kernel"


def _stats_of(trace: list[dict]) -> list[dict]:
    """Per-kernel rows in the form of rocprofv3's kernel_stats.csv (Name,
    Calls, AverageNs, MinNs, MaxNs, Percentage), by total time, from trace
    rows."""
    per: dict[str, list[int]] = {}
    for r in trace:
        per.setdefault(r["Kernel_Name"], []).append(
            int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    total = sum(sum(v) for v in per.values()) or 1
    rows = [{"Name": name, "Calls": len(v), "AverageNs": sum(v) / len(v), "MinNs": min(v),
             "MaxNs": max(v), "Percentage": 100.0 * sum(v) / total, "_total": sum(v)}
            for name, v in per.items()]
    return sorted(rows, key=lambda r: -r["_total"])


def summarize_trace(trace_dir: str, command: str | None = None,
                    title: str = "Qwen3-30B-A3B MoE layer, 64 tree tokens, 24-slot cache",
                    split: bool = True) -> str:
    """Kernel statistics of a ``rocprofv3 --kernel-trace --stats`` run of
    bench.py, with the K3 launch (gate/up + down pair) averages split into
    the in-step and all-resident phases at the calibration kernel."""
    stats_files = glob.glob(os.path.join(trace_dir, "**", "*kernel_stats.csv"), recursive=True)
    trace_files = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not stats_files or not trace_files:
        raise FileNotFoundError(f"no kernel stats/trace csv under {trace_dir}")
    with open(stats_files[0], newline="") as fh:
        stats = list(csv.DictReader(fh))
    with open(trace_files[0], newline="") as fh:
        trace = sorted(csv.DictReader(fh), key=lambda r: int(r["Start_Timestamp"]))
    lines = [f"# rocprofv3 kernel statistics — {title}", ""]
    if command:
        lines += ["Command (run from /tmp with TMPDIR=/tmp; `<repo>` is the repository root):", "",
                  "    " + command.replace("\n", "\n    "), ""]
    scope = "all dispatches of the process"
    if not split:
        # Workloads without the calibration kernel (the 48-layer forwards):
        # statistics from the first router launch on, so that set-up work
        # (drawing and encoding the expert sets) stays out of the table.
        first = next((i for i, r in enumerate(trace) if FORWARD_START in r["Kernel_Name"]), None)
        if first is not None:
            trace = trace[first:]
            stats = _stats_of(trace)
            scope = "every dispatch from the first router launch on"
    lines += [f"## Kernel statistics ({scope})", "",
              "| kernel | calls | avg µs | min µs | max µs | share |", "|---|---|---|---|---|---|"]
    for r in stats[:14]:
        name = r["Name"]
        short = name.replace("void ", "").replace("(anonymous namespace)::", "")
        if short.endswith(")"):  # drop the parameter list
            short = short[:short.rfind("(")]
        lines.append(f"| `{short[:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                     f"{float(r['Percentage']):.1f}% |")
    own = [r for r in stats if any(k in r["Name"] for k in LIBRARY_KERNELS)]
    if own:
        lines += ["", "## Kernels of libspecfit_amd (every instantiation)", "",
                  "| kernel | calls | avg µs | min µs | max µs | share |",
                  "|---|---|---|---|---|---|"]
        for r in own:
            short = r["Name"].replace("void ", "").replace("(anonymous namespace)::", "")
            if short.endswith(")"):
                short = short[:short.rfind("(")]
            lines.append(f"| `{short[:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                         f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                         f"{float(r['Percentage']):.1f}% |")
    cal = [i for i, r in enumerate(trace) if CALIBRATION_TAG in r["Kernel_Name"]]
    k3 = [(i, r) for i, r in enumerate(trace)
          if "gateup_mfma_kernel" in r["Kernel_Name"] or "down_mfma_kernel" in r["Kernel_Name"]]
    lines += ["", "## K3 launches (gate/up + down dispatch pairs)", "",
              "| phase | launches | avg gate/up µs | avg down µs | avg launch µs (sum) | "
              "avg weight MB | GB/s (weights / kernel time) |", "|---|---|---|---|---|---|---|"]
    phases = ((("in-step", [r for i, r in k3 if cal and i < cal[0]]),
               ("all-resident", [r for i, r in k3 if cal and i > cal[-1]])) if split
              else (("all", [r for _, r in k3]),))
    dur = lambda rs: sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rs) / len(rs) / 1e3
    for label, sel in phases:
        for table in (False, True):
            part = [r for r in sel if _is_table(r["Kernel_Name"]) == table]
            g = [r for r in part if "gateup" in r["Kernel_Name"]]
            d = [r for r in part if "down_mfma" in r["Kernel_Name"]]
            if not g or len(g) != len(d):
                continue
            t = dur(g) + dur(d)
            if table:  # the grid covers every table entry, not the experts computed
                lines.append(f"| {label}, slot table | {len(g)} | {dur(g):.2f} | {dur(d):.2f} | "
                             f"{t:.2f} | n/a | n/a |")
                continue
            wb = sum(_k3_weight_bytes(r["Kernel_Name"], int(r["Grid_Size_X"])) for r in part) / len(g)
            lines.append(f"| {label} | {len(g)} | {dur(g):.2f} | {dur(d):.2f} | {t:.2f} | "
                         f"{wb / 1e6:.2f} | {wb / (t * 1e-6) / 1e9:.0f} |")
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--fetch", help="rocprofv3 output dir of the FETCH_SIZE run")
    p.add_argument("--write", help="rocprofv3 output dir of the WRITE_SIZE run")
    p.add_argument("--trace", help="rocprofv3 output dir of a --kernel-trace --stats run")
    p.add_argument("--command", default=None, help="command lines to quote in the summary")
    p.add_argument("--out", default=None, help="write the markdown here (default: stdout)")
    p.add_argument("--title", default=None, help="workload named in the trace summary's title")
    p.add_argument("--no-split", action="store_true",
                   help="one K3 row over the whole trace (workloads without the calibration "
                        "kernel between phases)")
    args = p.parse_args(argv)
    if args.trace:
        kw = {"title": args.title} if args.title else {}
        text = summarize_trace(args.trace, args.command, split=not args.no_split, **kw)
    else:
        if not (args.fetch and args.write):
            p.error("--fetch and --write (or --trace) are required")
        text = summarize(args.fetch, args.write, args.command)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text)
    else:
        sys.stdout.write(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
