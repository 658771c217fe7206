#!/usr/bin/env python3
"""Benchmark of the offloaded Qwen3-MoE verification path on one MI355X.

Workload (default): one Qwen3-30B-A3B-shaped MoE layer (hidden 2048, 128
experts, top-8 renormalised softmax routing, intermediate 768, SwiGLU,
random-init N(0, 0.02) bf16 weights) verifying 64-token trees, with a
24-slot LRU GPU expert cache in front of all 128 experts held in pinned host
memory.  Router logits carry a seeded Zipf(s=1.1) popularity bias; the cache
is pre-warmed by 32 prior cycles (seeds 1-32).  A step is one MoE-layer
forward of a fresh 64-token batch (router K1 -> dispatch K2 -> cache
resolution + H2D -> grouped SwiGLU K3 -> combine K4), through the drop-in
runtime API (Qwen3MoeTopKRouterHip + Qwen3OffloadedExperts with the
resident-first policy and one-ahead prefetch).  Inputs are resident in HBM
before the timed region; the timed region includes every H2D transfer.  By
default a miss moves the expert's exponent-coded record (specfit_amd.codec,
~67% of the bytes), decoded into the slot on the device, which then holds
the raw bf16 bytes; --transfer raw moves the raw bytes, as the reference
does.

Every workload runs two passes of --steps steps.  The timed pass carries no
timing events: `value` and `ms_per_step` come from it.  The recorded pass,
over the next inputs, brackets every K3 launch (and each step's copy window)
with HIP events: the roofline, H2D, overlap and link-busy figures come from
it, and so do the per-step device times (K1 start to K4 end, H2D waits
included; median and 10th/90th percentile in `device_ms_per_step`).
--record none skips it.  Steps per pass default to 50 (10 for the 48-layer
forwards).  With --record copies the 48-layer recorded pass also times
every copy and marks every layer's router, and ``link`` splits the time the
host link idles into the gaps at layer boundaries (waiting for the next
layer's routing) and those inside a layer, with how long one or two copies
ran; those events slow the recorded pass, so its split is indicative.

The default single-layer run also reports, in the same line: a second
measurement of the same workload whose misses copy the raw bf16 expert bytes
as the reference does (``raw_transfer``), and shorter runs of the other
benchmark configurations (``other_configs``: 16 tokens all resident, the
1-128 token sweep, the 48-layer verification forward and the cold 128-token
forward, the last two also under the reference's ready_demand executor),
each exactly as its ``--workload`` run measures it, with fewer steps.

Prints ONE JSON line on stdout; diagnostics go to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

METRIC = ("verified tree tokens/s per MoE layer (1 GPU); achieved HBM GB/s + H2D GB/s")
HBM_PEAK_GBS = 8000.0
# Device sleep queued before each timed K3 launch of the recorded pass (about
# 25 us of shader clock), so a launch enqueued on an idle compute stream is
# timed from the device's start of the launch, not from the host's call.
PARK_CYCLES = 50_000


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None,
                   help="steps per pass (default 50; 10 for the 48-layer forwards)")
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--tokens", type=int, default=64)
    p.add_argument("--slots", type=int, default=24)
    p.add_argument("--prewarm", type=int, default=32)
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="budget of the CPU-baseline sample (0 disables it)")
    p.add_argument("--resident-reps", type=int, default=50)
    p.add_argument("--workload", choices=("layer", "resident16", "sweep", "verify48", "cold48"),
                   default="layer",
                   help="layer: one MoE layer, 64 tree tokens, 24-slot cache, Zipf routing (the "
                        "headline); resident16: 16 tokens, all 128 experts resident, uniform "
                        "routing; sweep: 1/8/32/64/128 tokens with a 12-slot cache; verify48: "
                        "the 48-layer verification forward of a 60-node depth-6 tree over a "
                        "1024-token context with 12-slot caches; cold48: the same forward with "
                        "128 tree tokens and every cache emptied before each forward")
    p.add_argument("--layers", type=int, default=48)
    p.add_argument("--context", type=int, default=1024)
    p.add_argument("--tree-nodes", type=int, default=60)
    p.add_argument("--tree-depth", type=int, default=6)
    p.add_argument("--verify-slots", type=int, default=12)
    p.add_argument("--transfer", choices=("raw", "coded"), default="coded",
                   help="what a miss moves over the host link: the expert's exponent-coded "
                        "record (specfit_amd.codec, ~67%% of the bytes, decoded into the slot "
                        "on the device; the slot holds the same bytes), or its raw bf16 bytes")
    p.add_argument("--expert-sets", type=int, default=24,
                   help="48-layer forwards: distinct pinned expert sets (1.125 GiB each); layer l "
                        "copies its misses from set l mod N.  The MI355X machines measured here "
                        "cap page-locked memory at ~36 GiB per process, so 48 distinct sets "
                        "(54 GiB) do not fit")
    p.add_argument("--shared-experts", action="store_true",
                   help="48-layer forwards: every layer's cache copies from one layer's pinned "
                        "experts, drawn on the host as in the single-layer workloads")
    p.add_argument("--executor", choices=("layer", "ready_demand", "predicted"), default="layer",
                   help="48-layer forwards only. layer: each MoE layer's own resident-first, "
                        "one-ahead sequence; ready_demand: the predicted-prefetch scheduler "
                        "(Qwen3ExpertPrefetch) with no predictions, the reference's measured "
                        "decode executor; predicted: the scheduler given each forward's own "
                        "routed experts as predictions (captured in untimed runs of the same "
                        "forwards before the warm-up: an upper bound for a draft's predictions)")
    p.add_argument("--lookahead", type=int, default=None,
                   help="the scheduler's lookahead_layers (default 0 for ready_demand, as the "
                        "reference's measured decode calls it; 1 for predicted)")
    p.add_argument("--max-inflight", type=int, default=2,
                   help="the scheduler's bound on incomplete transfers (default 2, the "
                        "reference's default)")
    p.add_argument("--no-raw-pass", dest="raw_pass", action="store_false",
                   help="single-layer workload with coded transfers: skip the second pass with "
                        "raw transfers (reported as raw_transfer)")
    p.add_argument("--no-other-configs", dest="other_configs", action="store_false",
                   help="single-layer workload: skip the shorter runs of the other "
                        "configurations (other_configs: resident16, sweep, verify48, cold48, "
                        "and the last two under the ready_demand executor)")
    p.add_argument("--config-steps", type=int, default=20,
                   help="steps per pass of the resident16 and sweep runs in other_configs")
    p.add_argument("--record", choices=("full", "k3", "none", "copies"), default="full",
                   help="timing events of the recorded pass: K3 launches + one copy window "
                        "per step (full), K3 only, or none (no recorded pass); copies (the "
                        "48-layer forwards): full plus an event pair around every copy and one "
                        "at every layer's router, for the link breakdown (the extra events slow "
                        "the recorded pass's host by 20-45%%)")
    args = p.parse_args(argv)
    if args.executor != "layer" and args.workload not in ("verify48", "cold48"):
        p.error("--executor applies to the 48-layer forwards (verify48, cold48)")
    if args.lookahead is None:
        args.lookahead = 1 if args.executor == "predicted" else 0
    if args.steps is None:
        args.steps = 10 if args.workload in ("verify48", "cold48") else 50
    return args


def step_stats(events) -> dict | None:
    """Median and 10th/90th percentile of per-step device times (ms) from
    (start, end) TimingEvent pairs recorded on the compute stream."""
    if not events:
        return None
    ms = sorted(a.elapsed_time(b) for a, b in events)
    pick = lambda q: ms[min(len(ms) - 1, int(q * (len(ms) - 1) + 0.5))]
    return {"median": pick(0.5), "p10": pick(0.1), "p90": pick(0.9), "n": len(ms)}


def cpu_baseline(layer, hidden_list, seconds: float) -> dict | None:
    """Time the CPU oracle (bf16 eager semantics of the reference layer) on
    a bounded sample of the same workload, on this host's cores."""
    if seconds <= 0:
        return None
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits

    import oracle

    import torch

    def bits(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    cores = len(os.sched_getaffinity(0))
    H, I, E, K = layer.hidden_size, layer.intermediate_size, layer.num_experts, layer.top_k
    t_conv = time.perf_counter()
    experts = {e: oracle.bf16_float(bits(layer.experts[e])) for e in range(E)}
    router_bits = bits(layer.router)
    log(f"cpu baseline: fp32 weight image built in {time.perf_counter() - t_conv:.1f}s")
    done_tokens = 0
    steps = 0
    with threadpool_limits(limits=cores):
        blas_threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
        host_inputs = [bits(h.cpu()) for h in hidden_list]
        start = time.perf_counter()
        while time.perf_counter() - start < seconds:
            hb = host_inputs[steps % len(host_inputs)]
            _, w_bits, idx, _ = oracle.router(hb, router_bits, K, True)
            oracle.moe_forward_bf16(oracle.bf16_float(hb), idx, oracle.bf16_float(w_bits),
                                    experts, H, I, E)
            done_tokens += hb.shape[0]
            steps += 1
        elapsed = time.perf_counter() - start
    return {"value": done_tokens / elapsed, "unit": "tokens/s", "cores": int(blas_threads),
            "kind": "port",
            "sample": (f"{steps} layer forwards x {hidden_list[0].shape[0]} tokens of the same "
                       f"workload ({elapsed:.1f}s): oracle router (C, 1 thread) + numpy bf16-eager "
                       f"expert loop (BLAS {blas_threads} threads) + C combine"),
            "cpu_model": _cpu_model()}


def decode_stats(rec) -> dict | None:
    """The coded-transfer decodes of a recorded pass: count, average
    event-bracketed duration on the copy stream (from the end of the
    record's copy to the end of the decode), and algorithmic bytes (record
    read + bf16 values written) over that time against the HBM peak."""
    if not rec.decodes:
        return None
    t = sum(s.elapsed_time(e) for _, _, s, e in rec.decodes) * 1e-3
    alg = sum(nbytes + 2 * n for nbytes, n, _, _ in rec.decodes)
    n = len(rec.decodes)
    return {"kernel": "decode_kernel (sf_expert_decode)", "count": n, "avg_us": t / n * 1e6,
            "alg_bytes_per_decode": alg / n, "gbs": alg / t / 1e9,
            "frac": alg / t / 1e9 / HBM_PEAK_GBS}


def _union_length(spans) -> float:
    total, cur_s, cur_e = 0.0, None, None
    for s_, e_ in sorted(spans):
        if cur_e is None or s_ > cur_e:
            if cur_e is not None:
                total += cur_e - cur_s
            cur_s, cur_e = s_, e_
        else:
            cur_e = max(cur_e, e_)
    if cur_e is not None:
        total += cur_e - cur_s
    return total


def link_stats(rec, step_events) -> dict | None:
    """Where the host link idles in the recorded 48-layer forwards, from a
    (start, end) event pair around every copy and an event at every layer's
    router.  Per forward: the union of the copy intervals, its gaps split
    into those that contain a router event of layers 1.. (the layer
    boundary: the link waits for the next layer's routing) and the rest
    (inside a layer), the time before the first copy and after the last
    one, and how long one copy or two copies at once were running."""
    if not rec.copy_spans or not rec.marks or not step_events:
        return None
    origin = step_events[0][0]
    t = lambda ev: origin.elapsed_time(ev) * 1e3  # us
    spans = sorted((t(a), t(b)) for a, b in rec.copy_spans)
    marks = [(label, t(ev)) for label, ev in rec.marks]
    steps = [(t(a), t(b)) for a, b in step_events]
    per = {"boundary_us": [], "boundary": 0.0, "within": 0.0, "prologue": 0.0, "epilogue": 0.0,
           "one": 0.0, "two": 0.0, "busy": 0.0}
    for s0, s1 in steps:
        sp = [c for c in spans if s0 <= c[0] < s1]
        if not sp:
            continue
        gaps, cur_e = [], sp[0][1]
        for a, b in sp[1:]:
            if a > cur_e:
                gaps.append((cur_e, a))
            cur_e = max(cur_e, b)
        per["prologue"] += sp[0][0] - s0
        per["epilogue"] += max(0.0, s1 - cur_e)
        bounds = [m for label, m in marks if s0 <= m < s1 and label != 0]
        at_boundary = set()
        for m in bounds:
            hit = next((g for g in gaps if g[0] <= m < g[1]), None)
            per["boundary_us"].append(0.0 if hit is None else hit[1] - hit[0])
            if hit is not None:
                at_boundary.add(hit)
        per["boundary"] += sum(b - a for a, b in at_boundary)
        per["within"] += sum(b - a for a, b in gaps if (a, b) not in at_boundary)
        edges = sorted([(a, 1) for a, _ in sp] + [(b, -1) for _, b in sp])
        active, last = 0, edges[0][0]
        for x, d in edges:
            if active == 1:
                per["one"] += x - last
            elif active >= 2:
                per["two"] += x - last
            if active:
                per["busy"] += x - last
            active, last = active + d, x
    n = len(steps)
    b = sorted(per["boundary_us"])
    return {"forwards": n, "copies": len(spans),
            "boundary_idle_us": {"median": b[len(b) // 2], "mean": sum(b) / len(b),
                                 "p90": b[min(len(b) - 1, 9 * len(b) // 10)],
                                 "boundaries": len(b)} if b else None,
            "ms_per_forward": {k: per[k] / n / 1e3 for k in
                               ("busy", "one", "two", "boundary", "within", "prologue",
                                "epilogue")}}


TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "k3_traffic_qwen3_layer_t64_slots24.md")


def _traffic_ratio() -> tuple[float | None, str | None]:
    """(FETCH + WRITE bytes) / expert-weight bytes of the in-step K3
    dispatches, from the committed counter summary of this workload; the
    per-launch traffic is this ratio times the launch's weight bytes."""
    try:
        with open(TRAFFIC_PROFILE) as fh:
            for line in fh:
                if line.startswith("traffic_ratio_in_step:"):
                    return float(line.split(":", 1)[1]), (
                        "profiles/k3_traffic_qwen3_layer_t64_slots24.md: scaled FETCH_SIZE + "
                        "WRITE_SIZE over expert-weight bytes of the in-step K3 dispatches, "
                        "times this run's weight bytes per launch")
    except OSError:
        pass
    return None, None


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main_verify(args) -> dict:
    """The 48-layer verification forward: per step, one target forward of
    [seed, 60 draft nodes] with the tree mask against a 1024-token context
    (then the context is cropped back), every MoE block offloaded with a
    12-slot cache and every attention layer on the HIP tree kernel."""
    import torch

    from specfit_amd import ops
    from specfit_amd.runtime import synthetic_tree, verify_draft_tree
    from specfit_amd.workloads import (make_kv_context, make_layer, make_layer_sources,
                                       make_verify_model)

    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    coded = args.transfer == "coded"
    if args.shared_experts:
        experts = make_layer(seed=0, pin_memory=True)
        expert_bytes = experts.expert_bytes
        loaded = make_verify_model(device=dev, layers=args.layers,
                                   slots_per_layer=args.verify_slots, experts=experts,
                                   compress_expert_sources=coded)
    else:
        n_src = min(args.layers, args.expert_sets)
        # Coded transfers copy from the page-locked records only, so the raw
        # sets can stay in pageable memory.
        sources = make_layer_sources(n_src, device=dev, seed=0, pin_memory=not coded)
        expert_bytes = sources[0].shape[1] * sources[0].element_size()
        log(f"{n_src} distinct expert sets drawn in {time.perf_counter() - t0:.1f}s "
            f"({sum(s.numel() for s in sources) * 2 / 2**30:.1f} GiB"
            f"{', pageable' if coded else ' pinned'})")
        loaded = make_verify_model(device=dev, layers=args.layers,
                                   slots_per_layer=args.verify_slots,
                                   layer_sources=[sources[l % n_src] for l in range(args.layers)],
                                   compress_expert_sources=coded)
    target = loaded.model
    config = target.config
    cache = make_kv_context(config, args.context, device=dev, seed=1)
    torch.cuda.synchronize()
    log(f"{args.layers}-layer target built in {time.perf_counter() - t0:.1f}s")
    recorded = args.record != "none"
    n = args.warmup + args.steps * (2 if recorded else 1)
    trees = [synthetic_tree(args.tree_nodes, args.tree_depth, seed=100 + i,
                            vocab=config.vocab_size) for i in range(n)]
    g = torch.Generator().manual_seed(5)
    seeds = [torch.randint(config.vocab_size, (1, 1), generator=g).to(dev) for _ in range(n)]

    cold = args.workload == "cold48"
    executor = args.executor
    predictions = [{} for _ in range(n)]
    if executor == "predicted":
        # Each forward's routed experts per layer, from the routers' outputs
        # (the triple's indices, as the reference's route capture reads
        # them) in an untimed run of the same forward from empty caches.
        routed = [set() for _ in target.model.layers]
        hooks = [layer.mlp.gate.register_forward_hook(
                     lambda mod, inp, out, ids=ids: ids.update(out[2].flatten().tolist()))
                 for layer, ids in zip(target.model.layers, routed)]
        try:
            with torch.inference_mode():
                for i in range(n):
                    for ids in routed:
                        ids.clear()
                    loaded.cold_reset_expert_caches()
                    verify_draft_tree(target, trees[i], seeds[i], cache, commit=False)
                    cache.crop(args.context)
                    predictions[i] = {l: tuple(sorted(ids)) for l, ids in enumerate(routed)}
        finally:
            for h in hooks:
                h.remove()
        # Routes do not depend on cache contents; start the measured
        # forwards from the empty caches every other executor starts from.
        loaded.cold_reset_expert_caches()
        log(f"captured the routed experts of {n} forwards")
    sched_stats = []

    def step(i):
        if executor == "layer":
            res = verify_draft_tree(target, trees[i], seeds[i], cache, commit=False)
        else:
            with loaded.prefetch_experts(predictions[i], lookahead_layers=args.lookahead,
                                         max_inflight=args.max_inflight) as sched:
                res = verify_draft_tree(target, trees[i], seeds[i], cache, commit=False)
            sched_stats.append(sched.stats())
        cache.crop(args.context)
        return res

    with torch.inference_mode():
        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()
        log("warm-up done")

        compute = torch.cuda.current_stream(dev)
        step_events = []

        def run_steps(first, recorder=None):
            """(wall seconds, misses, hits, accepted nodes) of steps first..+steps;
            with a recorder, a device-time event pair per step too."""
            wall = 0.0
            misses = hits = accepted = 0
            for i in range(first, first + args.steps):
                if cold:  # empty caches (this also clears their counters); not timed
                    loaded.cold_reset_expert_caches()
                before = [c.stats() for c in loaded.expert_caches]
                torch.cuda.synchronize()
                start = time.perf_counter()
                if recorder is not None:
                    ev = (ops.TimingEvent(), ops.TimingEvent())
                    ev[0].record(compute)
                accepted += len(step(i).accepted_node_ids)
                if recorder is not None:
                    recorder.close_copy_window()
                    ev[1].record(compute)
                    step_events.append(ev)
                torch.cuda.synchronize()
                wall += time.perf_counter() - start
                after = [c.stats() for c in loaded.expert_caches]
                misses += sum(a.h2d_submissions - b.h2d_submissions for a, b in zip(after, before))
                hits += sum(a.resident_hits - b.resident_hits for a, b in zip(after, before))
                log(f"step {i - first + 1}/{args.steps}" + (" (recorded)" if recorder else ""))
            return wall, misses, hits, accepted

        # Timed pass without timing events; recorded pass over the next trees.
        wall, misses, hits, accepted = run_steps(args.warmup)
        rec = ops.LaunchRecorder(copies=False)
        rec_wall, rec_misses = 0.0, 0
        if recorded:
            with ops.record_launches(copies=True, park_cycles=PARK_CYCLES,
                                     per_copy=args.record == "copies") as rec:
                marks = [layer.mlp.gate.register_forward_pre_hook(
                             lambda mod, inp, l=l: rec.mark(l, compute))
                         for l, layer in enumerate(target.model.layers)]
                try:
                    rec_wall, rec_misses, _, _ = run_steps(args.warmup + args.steps, rec)
                finally:
                    for h in marks:
                        h.remove()
    H = config.hidden_size
    k3 = [(nx, rows, tag, s_.elapsed_time(e_) * 1e-3) for nx, rows, tag, s_, e_ in rec.k3]
    k3_time = sum(x[3] for x in k3)
    k3_alg = sum(nx * expert_bytes + rows * H * 4 for nx, rows, _, _ in k3)
    h2d_time = rec.copy_busy_seconds() if rec.windows else 0.0
    q = 1 + args.tree_nodes
    value = args.steps * q / wall
    k3_achieved = k3_alg / k3_time / 1e9 if k3_time else 0.0
    line = {
        "metric": "verified tree tokens/s, 48-layer verification forward (1 GPU); achieved HBM "
                  "GB/s + H2D GB/s",
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": ("synthetic: random-init N(0,0.02) bf16 weights ("
                 + ("one layer's 128 experts shared by every layer's cache" if args.shared_experts
                    else f"{min(args.layers, args.expert_sets)} distinct expert sets "
                         f"({'their coded records' if coded else 'raw'} in pinned memory), layer "
                         f"l copies from set l mod {min(args.layers, args.expert_sets)}")
                 + f"), random N(0,1) {args.context}-token KV context, seeded random trees"),
        "config": {"workload": (f"qwen3-30b-a3b verification forward, {args.layers} layers, "
                                f"{args.tree_nodes}-node depth-{args.tree_depth} tree over a "
                                f"{args.context}-token context, {args.verify_slots}-slot LRU "
                                f"expert cache per layer" + (", caches emptied before every forward"
                                                      if cold else "")),
                   "layers": args.layers, "context": args.context, "tree_nodes": args.tree_nodes,
                   "tree_depth": args.tree_depth, "cache_slots": args.verify_slots,
                   "attention": "HIP tree attention (K5)",
                   "execution_policy": "resident_first", "h2d_prefetch": True,
                   "executor": executor, "transfer": args.transfer},
        "per_layer_tokens_per_s": value * args.layers,
        "roofline": {"bound": "hbm", "achieved": k3_achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": k3_achieved / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "K3 grouped SwiGLU (gateup_mfma + down_mfma dispatches)",
                     "launches": len(k3), "avg_launch_us": k3_time / max(len(k3), 1) * 1e6},
        "cpu_baseline": None,
        "recorded_ms_per_step": rec_wall / args.steps * 1e3 if rec_wall else None,
        "device_ms_per_step": step_stats(step_events),
        "h2d": {"achieved_gbs": rec.h2d_bytes / h2d_time / 1e9 if h2d_time else None,
                "expert_gbs": rec_misses * expert_bytes / h2d_time / 1e9 if h2d_time else None,
                "transfer": args.transfer,
                "transfers": rec_misses, "busy_ms": h2d_time * 1e3,
                "link_busy_frac": h2d_time / rec_wall if h2d_time else None},
        "cache": {"misses_per_layer": misses / (args.steps * args.layers),
                  "hits_per_layer": hits / (args.steps * args.layers)},
        "accepted_per_step": accepted / args.steps,
        "decode": decode_stats(rec),
        "link": link_stats(rec, step_events),
    }
    if sched_stats:  # the timed pass's forwards
        timed = sched_stats[args.warmup:args.warmup + args.steps]
        rows = [row for st in timed for row in st["layers"]]
        line["scheduler"] = {
            "lookahead_layers": args.lookahead, "max_inflight": args.max_inflight,
            "complete": all(st["complete"] for st in timed),
            "peak_inflight": max(st["peak_inflight"] for st in timed),
            "queue_capacity_waits": sum(st["queue_capacity_waits"] for st in timed) / len(timed),
            "slot_wait_copies": sum(st["slot_wait_copies"] for st in timed) / len(timed),
            "per_forward": {k: sum(r[k] for r in rows) / len(timed)
                            for k in ("predicted_experts", "actual_experts", "ready_at_router",
                                      "inflight_at_router", "missing_at_router",
                                      "prediction_copies", "demand_copies",
                                      "unused_prediction_copies", "compute_waits")}}
    loaded.close()
    return line


def main_sweep(args) -> dict:
    """Tree-size sweep: 1, 8, 32, 64 and 128 tokens through one Zipf-routed
    MoE layer with a 12-slot cache (the 32 pre-warm and the warm-up inputs
    cycled for at least 0.25 s before each point's timed pass)."""
    import torch

    from specfit_amd import ops
    from specfit_amd.runtime import (ExpertKey, GpuExpertCache, Qwen3MoeTopKRouterHip,
                                     Qwen3OffloadedExperts)
    from specfit_amd.workloads import make_hidden, make_layer

    dev = torch.device("cuda:0")
    layer = make_layer(seed=0, zipf_s=1.1, zipf_lambda=1.0, pin_memory=True)
    H, I, E, K = layer.hidden_size, layer.intermediate_size, layer.num_experts, layer.top_k
    router = Qwen3MoeTopKRouterHip(num_experts=E, hidden_size=H, top_k=K, norm_topk_prob=True,
                                   device=dev)
    with torch.no_grad():
        router.weight.copy_(layer.router)
    points = []
    slots = 12
    image = None
    if args.transfer == "coded":
        from specfit_amd.codec import CompressedExperts

        image = CompressedExperts.encode({ExpertKey(0, e): layer.experts[e] for e in range(E)},
                                         device=dev)
    for T in (1, 8, 32, 64, 128):
        cache = GpuExpertCache({ExpertKey(0, e): layer.experts[e] for e in range(E)},
                               slot_count=slots, device=dev, adopt_pinned_sources=True,
                               compressed_sources=image)
        experts = Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=H,
                                        intermediate_size=I, execution_policy="resident_first",
                                        h2d_prefetch=True)
        recorded = args.record != "none"
        n = args.prewarm + args.warmup + args.steps * (2 if recorded else 1)
        hidden = [make_hidden(T, H, seed=1 + i, zipf_fold=True).to(dev) for i in range(n)]

        def step(h):
            _, w, idx = router(h)
            return experts(h, idx, w), idx

        compute = torch.cuda.current_stream(dev)
        step_events = []

        def run_steps(inputs, recorder=None):
            """(wall seconds, misses, hits, routing indices) of one pass; with
            a recorder, a device-time event pair per step too."""
            before = cache.stats()
            idxs = []
            torch.cuda.synchronize()
            start = time.perf_counter()
            for h in inputs:
                if recorder is not None:
                    ev = (ops.TimingEvent(), ops.TimingEvent())
                    ev[0].record(compute)
                idxs.append(step(h)[1])
                if recorder is not None:
                    recorder.close_copy_window()
                    ev[1].record(compute)
                    step_events.append(ev)
            torch.cuda.synchronize()
            wall = time.perf_counter() - start
            after = cache.stats()
            return (wall, after.h2d_submissions - before.h2d_submissions,
                    after.resident_hits - before.resident_hits, idxs)

        # Pre-warm and warm-up inputs, cycled until at least 0.25 s of steps
        # have run: a 1-token step takes ~0.4 ms, and the first point of a
        # process otherwise starts timing before the device has left idle.
        base = args.prewarm + args.warmup
        torch.cuda.synchronize()
        warm_start = time.perf_counter()
        while True:
            for i in range(base):
                step(hidden[i])
            torch.cuda.synchronize()
            if time.perf_counter() - warm_start >= 0.25:
                break
        # Timed pass without timing events; recorded pass over the next inputs.
        wall, misses, hits, idxs = run_steps(hidden[base:base + args.steps])
        rec = ops.LaunchRecorder(copies=False)
        rec_wall, rec_misses = 0.0, 0
        if recorded:
            with ops.record_launches(copies=args.record in ("full", "copies"), park_cycles=PARK_CYCLES) as rec:
                rec_wall, rec_misses, _, _ = run_steps(hidden[base + args.steps:], rec)
        ms = []
        for idx in idxs:
            counts = torch.bincount(idx.reshape(-1).cpu(), minlength=E)
            ms.extend(int(c) for c in counts if c > 0)
        k3 = [(nx, rows, s_.elapsed_time(e_) * 1e-3) for nx, rows, _, s_, e_ in rec.k3]
        k3_time = sum(x[2] for x in k3)
        k3_bytes = sum(nx * layer.expert_bytes + rows * H * 4 for nx, rows, _ in k3)
        k3_weight = sum(nx * layer.expert_bytes for nx, _, _ in k3)
        k3_flops = sum(2 * rows * 3 * H * I for _, rows, _ in k3)
        h2d_time = rec.copy_busy_seconds() if rec.windows else 0.0
        points.append({
            "tokens": T, "tokens_per_s": args.steps * T / wall,
            "ms_per_step": wall / args.steps * 1e3,
            "recorded_ms_per_step": rec_wall / args.steps * 1e3 if rec_wall else None,
            "device_ms_per_step": step_stats(step_events),
            "misses_per_step": misses / args.steps,
            "hits_per_step": hits / args.steps,
            "distinct_experts_per_step": len(ms) / args.steps,
            "rows_per_expert": {"mean": sum(ms) / len(ms), "max": max(ms)},
            "k3_flop_per_weight_byte": k3_flops / k3_weight if k3_weight else None,
            "k3_gbs": k3_bytes / k3_time / 1e9 if k3_time else None,
            "k3_frac": k3_bytes / k3_time / 1e9 / HBM_PEAK_GBS if k3_time else None,
            "h2d_gbs": rec.h2d_bytes / h2d_time / 1e9 if h2d_time else None,
            "h2d_expert_gbs": (rec_misses * layer.expert_bytes / h2d_time / 1e9
                               if h2d_time else None),
            "h2d_link_busy_frac": h2d_time / rec_wall if h2d_time else None,
            "decode": decode_stats(rec),
        })
        log(f"T={T}: {points[-1]['tokens_per_s']:.0f} tokens/s, "
            f"{points[-1]['misses_per_step']:.2f} misses/step")
        cache.close()
    line = {"metric": "verified tree tokens/s per MoE layer across tree sizes (1 GPU)",
            "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "dtype": "bf16", "data": "synthetic (as the layer workload)",
            "config": {"workload": "qwen3-30b-a3b moe layer, 12-slot LRU cache, zipf 1.1, "
                                   "prewarm 32 cycles repeated for >= 0.25 s, tokens 1/8/32/64/128",
                       "cache_slots": slots, "prewarm_cycles": args.prewarm,
                       "transfer": args.transfer},
            "points": points}
    return line


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(the verification path runs on a single MI355X; multi-GPU sharding is a "
              "design note, not a built path)", file=sys.stderr)
        return 2
    import torch

    # Verification needs no autograd: every workload runs under inference
    # mode, as the reference's measured decode loop does
    # (scripts/run_specfit_main_comparison.py:713).
    with torch.inference_mode():
        line = main_workload(args)
        if args.workload == "layer" and args.other_configs:
            line["other_configs"] = other_configs(args)
    print(json.dumps(line), flush=True)
    return 0


def _config_run(argv: list[str], pick) -> dict:
    """One more workload in this process (its own inputs, cache and model,
    freed afterwards); ``pick`` keeps the figures the summary reports.  A
    failure is reported in the summary instead of ending the run."""
    import gc

    import torch

    log(f"other configuration: {' '.join(argv)}")
    try:
        out = pick(main_workload(parse_args(argv)))
    except Exception as exc:  # noqa: BLE001 - reported, not raised
        out = {"error": f"{type(exc).__name__}: {exc}"}
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    out["command"] = "python bench.py " + " ".join(argv)
    return out


def other_configs(args) -> dict:
    """The other benchmark configurations, each in a shorter run of its own
    (fewer steps; the same code path as ``--workload``):
    16 tokens all resident; the 1-128 token sweep; the 48-layer
    verification forward and the cold 128-token forward, each with the
    per-layer executor and with the reference's ready_demand executor."""
    steps, tr = str(args.config_steps), ["--transfer", args.transfer]
    # The 48-layer runs take the forward's shape options of this run.
    shape = ["--layers", str(args.layers), "--context", str(args.context),
             "--verify-slots", str(args.verify_slots), "--expert-sets", str(args.expert_sets)]

    def layer_pick(d):
        return {"value": d["value"], "unit": d["unit"], "ms_per_step": d["ms_per_step"],
                "workload": d["config"]["workload"], "k3_frac": d["roofline"]["frac"],
                "k3_gbs": d["roofline"]["achieved"],
                "cpu_baseline": d["cpu_baseline"] and {k: d["cpu_baseline"][k]
                                                       for k in ("value", "unit", "cores")}}

    def sweep_pick(d):
        keep = ("tokens", "tokens_per_s", "ms_per_step", "misses_per_step", "k3_gbs",
                "h2d_expert_gbs", "h2d_link_busy_frac")
        return {"workload": d["config"]["workload"], "transfer": d["config"]["transfer"],
                "points": [{k: p[k] for k in keep} for p in d["points"]]}

    def verify_pick(d):
        return {"value": d["value"], "unit": d["unit"], "ms_per_step": d["ms_per_step"],
                "workload": d["config"]["workload"], "transfer": d["config"]["transfer"],
                "executor": d["config"]["executor"],
                "per_layer_tokens_per_s": d["per_layer_tokens_per_s"],
                "misses_per_layer": d["cache"]["misses_per_layer"]}

    verify_args = ["--workload", "verify48", "--steps", "5", "--warmup", "2", "--record", "none",
                   "--tree-nodes", str(args.tree_nodes), *shape, *tr]
    cold_args = ["--workload", "cold48", "--steps", "5", "--warmup", "2", "--record", "none",
                 *shape, *tr]
    # The same forwards under the reference's measured decode executor (the
    # prefetch scheduler with no predictions, lookahead 0, two credits).
    rd = ["--executor", "ready_demand"]

    return {
        "resident16": _config_run(["--workload", "resident16", "--steps", steps, "--warmup", "5",
                                   "--cpu-seconds", "2", "--record", "k3"], layer_pick),
        "sweep": _config_run(["--workload", "sweep", "--steps", steps, "--warmup", "5",
                              "--record", "k3", *tr], sweep_pick),
        "verify48": _config_run(verify_args, verify_pick),
        "cold48": _config_run(cold_args, verify_pick),
        "verify48_ready_demand": _config_run(verify_args + rd, verify_pick),
        "cold48_ready_demand": _config_run(cold_args + rd, verify_pick),
    }


def _layer_pass(args, dev, layer, router, hidden, image, *, resident: bool) -> dict:
    """One measurement of the single-layer workload on a fresh cache:
    pre-warm (``args.prewarm`` cycles), warm-up, a timed pass of
    ``args.steps`` steps without timing events, then (unless ``--record
    none``) a recorded pass over the next inputs with HIP events around
    every K3 launch and copy window.  ``image`` selects coded transfers
    (None: raw bytes)."""
    import torch

    from specfit_amd import ops
    from specfit_amd.runtime import ExpertKey, GpuExpertCache, Qwen3OffloadedExperts

    H, I, E = layer.hidden_size, layer.intermediate_size, layer.num_experts
    cache = GpuExpertCache({ExpertKey(0, e): layer.experts[e] for e in range(E)},
                           slot_count=args.slots, device=dev, adopt_pinned_sources=True,
                           cache_id="qwen3-layer-0", queue_id="layer-0-copy",
                           compressed_sources=image)
    experts = Qwen3OffloadedExperts(layer_id=0, cache=cache, hidden_size=H, intermediate_size=I,
                                    execution_policy="resident_first", h2d_prefetch=True)

    def step(h):
        _, w, idx = router(h)
        return experts(h, idx, w)

    if resident:  # every expert in its own slot before the first step
        for e in range(E):
            with cache.acquire(ExpertKey(0, e)) as lease:
                lease.wait()
    # Pre-warm the cache with the prior cycles, then untimed warm-up steps.
    for i in range(args.prewarm):
        step(hidden[i])
    torch.cuda.synchronize()
    log(f"prewarmed {args.prewarm} cycles ({'coded' if image is not None else 'raw'}); "
        f"cache stats {cache.stats()}")
    for i in range(args.warmup):
        step(hidden[args.prewarm + i])
    torch.cuda.synchronize()

    compute = torch.cuda.current_stream(dev)
    step_events = []

    def run_steps(inputs, recorder=None):
        """(wall seconds, misses, hits) of one pass over ``inputs``; with a
        recorder, also a device-time event pair per step (K1 start .. K4
        end, H2D waits included) into ``step_events``."""
        before = cache.stats()
        torch.cuda.synchronize()
        start = time.perf_counter()
        for h in inputs:
            if recorder is not None:
                ev = (ops.TimingEvent(), ops.TimingEvent())
                ev[0].record(compute)
            step(h)
            if recorder is not None:
                recorder.close_copy_window()
                ev[1].record(compute)
                step_events.append(ev)
        torch.cuda.synchronize()
        wall = time.perf_counter() - start
        after = cache.stats()
        return (wall, after.h2d_submissions - before.h2d_submissions,
                after.resident_hits - before.resident_hits)

    # Timed pass: no timing events, so `value` is the uninstrumented path.
    base = args.prewarm + args.warmup
    timed = hidden[base:base + args.steps]
    wall, misses, hits = run_steps(timed)
    log(f"timed {args.steps} steps in {wall * 1e3:.2f} ms: {misses} misses, {hits} hits")
    # Recorded pass over the next inputs: HIP events around every K3 launch
    # (and every copy window) give the roofline, H2D and overlap figures.
    rec = ops.LaunchRecorder(copies=False)
    rec_wall, rec_misses = 0.0, 0
    if args.record != "none":
        with ops.record_launches(copies=args.record in ("full", "copies"), park_cycles=PARK_CYCLES) as rec:
            rec_wall, rec_misses, _ = run_steps(hidden[base + args.steps:], rec)
        log(f"recorded {args.steps} steps in {rec_wall * 1e3:.2f} ms: {rec_misses} misses")
    torch.cuda.synchronize()
    cache.close()
    return dict(timed=timed, wall=wall, misses=misses, hits=hits, rec=rec, rec_wall=rec_wall,
                rec_misses=rec_misses, step_events=step_events)


def _pass_figures(p: dict, k3_bytes, expert_bytes: int) -> dict:
    """K3, H2D and overlap figures of a recorded pass from ``_layer_pass``."""
    rec = p["rec"]
    # K3 (grouped SwiGLU gate/up + down dispatches) over the recorded pass.
    k3 = [(n, rows, tag, s.elapsed_time(e) * 1e-3) for n, rows, tag, s, e in rec.k3]
    res = [x for x in k3 if x[2] == "resident"]
    h2d_time = rec.copy_busy_seconds() if rec.windows else 0.0
    # Overlap of transfers and expert GEMMs: (t_h2d + t_gemm - t_union) /
    # min(t_h2d, t_gemm), with t_union the measured union of the copy windows
    # and the K3 launch intervals (all events share the device clock).
    overlap = None
    if rec.windows and rec.k3:
        origin = rec.windows[0][0]
        spans_copy = [(origin.elapsed_time(a), origin.elapsed_time(b)) for a, b in rec.windows]
        spans_k3 = [(origin.elapsed_time(a), origin.elapsed_time(b)) for *_, a, b in rec.k3]
        t_union = _union_length(spans_copy + spans_k3) * 1e-3
        t_gemm = _union_length(spans_k3) * 1e-3
        t_h2d = _union_length(spans_copy) * 1e-3
        overlap = max(0.0, min(1.0, (t_h2d + t_gemm - t_union) / min(t_h2d, t_gemm)))
    # K3 launches that ran beside a decode (their event intervals intersect
    # one of the recorded decodes') against those that ran alone.
    beside = None
    if rec.k3 and rec.decodes:
        origin = rec.k3[0][3]
        spans_dec = sorted((origin.elapsed_time(a), origin.elapsed_time(b))
                           for *_, a, b in rec.decodes)
        groups = {"beside_decode": [0, 0, 0.0], "alone": [0, 0, 0.0]}
        for (n, rows, _, sec), (*_, a, b) in zip(k3, rec.k3):
            s0, s1 = origin.elapsed_time(a), origin.elapsed_time(b)
            hit = any(d0 < s1 and d1 > s0 for d0, d1 in spans_dec)
            g = groups["beside_decode" if hit else "alone"]
            g[0] += 1
            g[1] += k3_bytes(n, rows)
            g[2] += sec
        beside = {k: {"launches": v[0], "gbs": v[1] / v[2] / 1e9 if v[2] else None}
                  for k, v in groups.items()}
    return dict(k3=k3, k3_time=sum(x[3] for x in k3), k3_beside_decode=beside,
                k3_alg=sum(k3_bytes(n, r) for n, r, _, _ in k3), res=res,
                res_bytes=sum(k3_bytes(n, r) for n, r, _, _ in res),
                res_time=sum(x[3] for x in res),
                h2d_bytes=rec.h2d_bytes,  # over the link (coded records or raw experts)
                h2d_expert_bytes=p["rec_misses"] * expert_bytes, h2d_time=h2d_time,
                overlap=overlap)


def main_workload(args) -> dict:
    """Run the workload ``args`` names and return its JSON line."""
    if args.workload in ("verify48", "cold48"):
        if args.workload == "cold48" and args.tree_nodes == 60:
            args.tree_nodes = 127  # 128 tree tokens
        return main_verify(args)
    if args.workload == "sweep":
        return main_sweep(args)
    if args.workload == "resident16":
        args.tokens, args.slots = 16, 128

    import torch

    from specfit_amd import ops
    from specfit_amd.codec import CompressedExperts
    from specfit_amd.runtime import ExpertKey, Qwen3MoeTopKRouterHip
    from specfit_amd.workloads import make_hidden, make_layer

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a HIP device")
    dev = torch.device("cuda:0")
    T, slots = args.tokens, args.slots
    resident = args.workload == "resident16"
    t0 = time.perf_counter()
    layer = make_layer(seed=0, zipf_s=None if resident else 1.1, zipf_lambda=1.0,
                       pin_memory=True)
    H, I, E, K = layer.hidden_size, layer.intermediate_size, layer.num_experts, layer.top_k
    expert_bytes = layer.expert_bytes
    log(f"layer generated in {time.perf_counter() - t0:.1f}s "
        f"({E} experts x {expert_bytes} B pinned)")

    router = Qwen3MoeTopKRouterHip(num_experts=E, hidden_size=H, top_k=K, norm_topk_prob=True,
                                   device=dev)
    with torch.no_grad():
        router.weight.copy_(layer.router)
    image = None
    if args.transfer == "coded":
        t1 = time.perf_counter()
        image = CompressedExperts.encode({ExpertKey(0, e): layer.experts[e] for e in range(E)},
                                         device=dev)
        log(f"experts coded in {time.perf_counter() - t1:.1f}s: {image.transfer_bytes} of "
            f"{image.raw_bytes} B ({image.transfer_bytes / image.raw_bytes:.4f})")
    n_inputs = args.prewarm + args.warmup + args.steps * (1 if args.record == "none" else 2)
    hidden = [make_hidden(T, H, seed=(0 if resident else 1) + i, zipf_fold=not resident).to(dev)
              for i in range(n_inputs)]
    torch.cuda.synchronize()

    def k3_bytes(n, rows):
        # expert weights + gathered hidden rows read + weighted rows written
        return n * expert_bytes + rows * H * 2 * 2

    p = _layer_pass(args, dev, layer, router, hidden, image, resident=resident)
    rec, timed = p["rec"], p["timed"]
    wall, misses, hits = p["wall"], p["misses"], p["hits"]
    f = _pass_figures(p, k3_bytes, expert_bytes)
    k3, k3_alg, k3_time = f["k3"], f["k3_alg"], f["k3_time"]
    res_bytes, res_time, res = f["res_bytes"], f["res_time"], f["res"]
    h2d_bytes, h2d_expert_bytes, h2d_time = f["h2d_bytes"], f["h2d_expert_bytes"], f["h2d_time"]
    rec_wall, rec_misses, overlap = p["rec_wall"], p["rec_misses"], f["overlap"]
    step_events = p["step_events"]

    # The reference's transfer semantics beside the coded headline: a fresh
    # cache whose misses move the raw bf16 expert bytes, the same pre-warm
    # and the same inputs.
    raw_pass = None
    if image is not None and not resident and args.raw_pass:
        q = _layer_pass(args, dev, layer, router, hidden, None, resident=False)
        g = _pass_figures(q, k3_bytes, expert_bytes)
        raw_pass = {
            "value": args.steps * T / q["wall"], "unit": "tokens/s",
            "ms_per_step": q["wall"] / args.steps * 1e3,
            "misses_per_step": q["misses"] / args.steps,
            "hits_per_step": q["hits"] / args.steps,
            "h2d_gbs": g["h2d_bytes"] / g["h2d_time"] / 1e9 if g["h2d_time"] else None,
            "h2d_link_busy_frac": g["h2d_time"] / q["rec_wall"] if g["h2d_time"] else None,
            "overlap": g["overlap"],
            "k3_in_step_gbs": g["k3_alg"] / g["k3_time"] / 1e9 if g["k3_time"] else None,
            "k3_in_step_frac": (g["k3_alg"] / g["k3_time"] / 1e9 / HBM_PEAK_GBS
                                if g["k3_time"] else None),
            "k3_resident_in_step_gbs": (g["res_bytes"] / g["res_time"] / 1e9
                                        if g["res_time"] else None),
            "note": ("same workload, inputs and pre-warm with a fresh cache whose misses copy "
                     "the raw bf16 expert bytes (9,437,184 B each), as the reference does"),
        }
        log(f"raw-transfer pass: {raw_pass['value']:.0f} tokens/s, "
            f"{raw_pass['ms_per_step']:.3f} ms/step")

    # A plain elementwise kernel of known size (256 MiB read + 256 MiB
    # written).  Under rocprofv3 --pmc it calibrates FETCH_SIZE / WRITE_SIZE
    # and separates the in-step K3 dispatches from the all-resident ones
    # (specfit_amd/pmc.py).
    cal_src = torch.ones((256 << 20) // 4, dtype=torch.float32, device=dev)
    cal_dst = torch.empty_like(cal_src)
    torch.neg(cal_src, out=cal_dst)
    torch.cuda.synchronize()
    del cal_src, cal_dst

    # Host-link peak: best of 10 x 1 GiB pinned -> device copies.
    flat = layer.experts.view(-1)
    gib = 1 << 30
    src = flat[: gib // 2]
    dst = torch.empty(gib // 2, dtype=torch.bfloat16, device=dev)
    side = torch.cuda.Stream(device=dev)
    best = 0.0
    for _ in range(10):
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_ev.record(side)
        ops.copy_h2d(dst, src, side)
        e_ev.record(side)
        e_ev.synchronize()
        best = max(best, gib / (s_ev.elapsed_time(e_ev) * 1e-3) / 1e9)
    del dst
    log(f"host link peak {best:.1f} GB/s; h2d achieved "
        f"{(h2d_bytes / h2d_time / 1e9) if h2d_time else 0:.1f} GB/s")

    # Resident-expert GEMM: K3 over every active expert of a 64-token Zipf
    # batch with all experts resident in HBM (the all-resident case).
    all_slots = layer.experts.to(dev)
    h = hidden[-1]
    _, w, idx = router(h)
    plan = ops.dispatch(idx, E)
    active = plan.active_experts()
    counts = plan.fetch_counts()[0]
    rows_n = int(sum(int(counts[e]) for e in active))
    act = torch.empty((T * K, I), dtype=torch.bfloat16, device=dev)
    rows = torch.empty((T * K, H), dtype=torch.bfloat16, device=dev)
    wflat = w.reshape(-1).contiguous()
    weights = [all_slots[e] for e in active]
    for _ in range(5):
        ops.grouped_swiglu(h, plan, wflat, active, weights, H, I, act, rows)
    torch.cuda.synchronize()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_ev.record()
    for _ in range(args.resident_reps):
        ops.grouped_swiglu(h, plan, wflat, active, weights, H, I, act, rows)
    e_ev.record()
    e_ev.synchronize()
    res_launch = s_ev.elapsed_time(e_ev) * 1e-3 / args.resident_reps
    res_launch_bytes = k3_bytes(len(active), rows_n)
    log(f"all-resident K3: {len(active)} experts, {rows_n} rows, {res_launch * 1e6:.1f} us, "
        f"{res_launch_bytes / res_launch / 1e9:.0f} GB/s")
    del all_slots

    cpu = cpu_baseline(layer, timed, args.cpu_seconds)

    value = args.steps * T / wall
    k3_achieved = k3_alg / k3_time / 1e9 if k3_time else 0.0
    ratio, ratio_src = _traffic_ratio() if not resident else (None, None)
    k3_weight_per_launch = sum(n for n, *_ in k3) * expert_bytes / max(len(k3), 1)
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": ("synthetic: seeded N(0,1) hidden states, router and experts random-init "
                 "N(0,0.02) bf16" + ("" if resident else ", Zipf(1.1)-biased routing")),
        "config": {"workload": ("qwen3-30b-a3b moe layer verify, 16 tree tokens, all 128 experts "
                                "resident in HBM, uniform routing" if resident else
                                f"qwen3-30b-a3b moe layer verify, {T} tree tokens, {slots}-slot "
                                f"LRU expert cache, 128 experts in pinned host memory, zipf 1.1, "
                                f"prewarm {args.prewarm} cycles"),
                   "tokens": T, "hidden": H, "experts": E, "top_k": K, "intermediate": I,
                   "cache_slots": slots, "prewarm_cycles": args.prewarm,
                   "execution_policy": "resident_first", "h2d_prefetch": True,
                   "transfer": args.transfer},
        "record": args.record,
        "recorded_ms_per_step": rec_wall / args.steps * 1e3 if rec_wall else None,
        "device_ms_per_step": step_stats(step_events),
        "roofline": {"bound": "hbm", "achieved": k3_achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": k3_achieved / HBM_PEAK_GBS,
                     "traffic": ratio * k3_weight_per_launch if ratio and k3 else None,
                     "traffic_source": ratio_src,
                     "kernel": "K3 grouped SwiGLU (gateup_mfma + down_mfma dispatches)",
                     "launches": len(k3), "avg_launch_us": k3_time / max(len(k3), 1) * 1e6,
                     "alg_bytes_per_launch": k3_alg / max(len(k3), 1)},
        "cpu_baseline": cpu,
        "h2d": {"achieved_gbs": h2d_bytes / h2d_time / 1e9 if h2d_time else None,
                "expert_gbs": h2d_expert_bytes / h2d_time / 1e9 if h2d_time else None,
                "transfer": args.transfer,
                "bytes_note": "bytes: moved over the host link (coded records, or raw experts); "
                              "expert_bytes: the bf16 expert bytes those transfers delivered to "
                              "HBM",
                "link_peak_gbs": best, "transfers": rec_misses, "bytes": h2d_bytes,
                "expert_bytes": h2d_expert_bytes,
                "busy_ms": h2d_time * 1e3,
                "note": "busy = union over steps of [first copy start, last copy end] on the two "
                        "copy streams"},
        "cache": {"misses_per_step": misses / args.steps, "hits_per_step": hits / args.steps},
        "overlap": overlap,
        "h2d_link_busy_frac": h2d_time / rec_wall if h2d_time else None,
        "decode": decode_stats(rec),
        "k3_resident_in_step": {"launches": len(res),
                                "gbs": res_bytes / res_time / 1e9 if res_time else None},
        "k3_in_step_by_decode_overlap": f["k3_beside_decode"],
        "k3_all_resident": {"experts": len(active), "rows": rows_n, "us": res_launch * 1e6,
                            "gbs": res_launch_bytes / res_launch / 1e9,
                            "frac": res_launch_bytes / res_launch / 1e9 / HBM_PEAK_GBS},
    }
    if raw_pass is not None:
        line["raw_transfer"] = raw_pass
    return line


if __name__ == "__main__":
    sys.exit(main())
