"""Benchmark of the restricted decode tail on one MI355X.

Workload cfg3: a continuous-batching pack of
B = 256 sequences over the 49152 x 576 FP16 tied embedding; allowed-set sizes
log-uniform in [1, 4096]; 10% of rows unrestricted (MFMA fallback); hidden
N(0, 1) through the final RMSNorm.  Synthetic data (seeded), inputs resident
in HBM before the timed region.

One step = one mf_decode_tail_f16 call over the whole pack: RMSNorm and the
range index of each row's (ascending) list, one pass over the table scoring
the restricted rows' candidates and the unrestricted rows on MFMA,
DFA/selection outputs.  Eight copies of the embedding (453 MB > the 256 MiB
Infinity Cache) are rotated so no step finds the table cached by the previous
one.

The GPU's clocks ramp up under load: a short run straight after the set-up
(which leaves the compute units idle) measures 3-4% slower than the steady
state of a decode loop.  Before the --warmup steps the step therefore runs,
untimed, for --device-warmup-ms of wall time (default 100 ms); the line
reports it as device_warmup_ms, and the timed region is still exactly
--steps steps.

Prints one JSON line: metric/value (sequences per second), the roofline of
the dominant kernel (the table pass) from HIP events on its stream, the same
step on the gather + MFMA head kernels, the full-vocabulary comparator
("x vs full head"), and the CPU oracle timed on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
METRIC = "restricted-head seqs/sec + % HBM roofline @B=256 ragged; x vs full head"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--config", type=int, default=3, help="benchmark configuration cfgN")
    p.add_argument("--copies", type=int, default=8)
    p.add_argument("--device-warmup-ms", type=float, default=100.0,
                   help="untimed steps for this long before --warmup (clock ramp)")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="budget of the CPU oracle baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-full", action="store_true")
    p.add_argument("--no-gather-path", action="store_true",
                   help="skip timing the same step on the gather + MFMA head kernels")
    p.add_argument("--no-reference-bench", action="store_true",
                   help="skip the reference's 12-cell output-head benchmark")
    p.add_argument("--calibration-copy-mib", type=int, default=0,
                   help="after the timed loop, run 4 FP32 x1.0 copies of this many MiB "
                        "(a known-traffic kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return p.parse_args()


def algorithmic_bytes(w) -> dict:
    """Bytes one launch must move:
    gather   2 H U + 4 N + 4 H B_r + 4 (B_r + 1) + 12 B_r
    fallback 2 V H + 4 H B_u + 8 B_u, flops 2 B_u H V
    pass     2 H T + 4 N + 4 H B + 4 (B_r + 1) + 12 B with T = V when there
             are unrestricted rows (the table is read once for both kinds of
             rows), else U; flops 2 (B_u H V + N H) (candidates and the
             unrestricted rows' head, FP16 hi of z)
    dense    2 V H + 2 H S with S = B_u + D slots (D: the longest lists
             of at least max(64, V / 256) ids, as many as fill the room the
             B_u rows leave in their panels of 256 slots, then whole panels
             while a panel's lists hold 5 V / 2 ids); flops 2 S H V; the
             gather then moves the other restricted rows' bytes
             (gather_rest: their distinct ids' rows; gather_rest_logical:
             every candidate's row, the bytes its waves fetch)."""
    H, V = w.hidden, w.vocab
    counts = w.row_counts()
    restricted = w.row_state < w.states
    B_r = int(restricted.sum())
    B_u = int((w.row_state == 0xFFFFFFFE).sum())
    N = int(counts[restricted].sum())
    U = w.distinct_restricted_ids()
    gather = 2 * H * U + 4 * N + 4 * H * B_r + 4 * (B_r + 1) + 12 * B_r
    logical = 2 * H * N + 4 * N + 4 * H * B_r + 4 * (B_r + 1) + 12 * B_r
    B = w.rows
    T = V if B_u > 0 else U
    dense_min = max(64, V // 256)
    cand = np.nonzero(restricted & (counts >= dense_min))[0]
    order = cand[np.lexsort((cand, -counts[cand]))]  # longest first, then by row
    D = min(-(-B_u // 256) * 256 - B_u, order.size)
    while D < order.size and int(counts[order[D:D + 256]].sum()) >= 5 * V // 2:
        D = min(D + 256, order.size)
    dense_rows = np.zeros(restricted.shape, bool)
    dense_rows[order[:D]] = True
    S = B_u + D
    rest = restricted & ~dense_rows
    N_rest = int(counts[rest].sum())
    U_rest = w.distinct_restricted_ids(rest)
    B_rest = int(rest.sum())
    gather_rest = 2 * H * U_rest + 4 * N_rest + 4 * H * B_rest + 4 * (B_rest + 1) + 12 * B_rest
    # the same with every candidate's row (a duplicate id read once per row)
    gather_rest_logical = (2 * H * N_rest + 4 * N_rest + 4 * H * B_rest + 4 * (B_rest + 1) +
                           12 * B_rest)
    return dict(gather=gather, gather_logical=logical, N=N, U=U, B_r=B_r, B_u=B_u,
                D=D, dense_bytes=2 * V * H + 2 * H * S, dense_flops=2 * S * H * V,
                gather_rest=gather_rest, gather_rest_logical=gather_rest_logical,
                B_rest=B_rest,
                fallback_bytes=2 * V * H + 4 * H * B_u + 8 * B_u,
                fallback_flops=2 * B_u * H * V,
                pass_bytes=2 * H * T + 4 * N + 4 * H * B + 4 * (B_r + 1) + 12 * B,
                pass_flops=2 * (B_u * H * V + N * H))


def time_loop(tail, stages, steps, warmup, copies):
    """Runs `steps` steps (after `warmup`), bracketed by synchronization.
    Returns the HIP-event ms per step (two events around the whole loop),
    the wall ms per step and, with more than one stage, each stage's mean
    and median ms from events recorded between the stages (those per-stage
    events are only recorded for multi-stage loops: an event record costs
    a few microseconds of stream time, which would inflate a one-stage
    step)."""
    import torch
    from market_sim_amd import abi, ops

    fns = {"prepare": ops.decode_tail_prepare, "restricted": ops.decode_tail_restricted,
           "unrestricted": ops.decode_tail_unrestricted,
           "finalize": ops.decode_tail_finalize, "full": ops.decode_tail_full_f16,
           "tail": ops.decode_tail_f16}
    args = [tail.args(i % copies) for i in range(copies)]
    s = tail.stream
    handle = s.cuda_stream
    for i in range(warmup):
        for st in stages:
            abi.check(st, fns[st](args[i % copies], handle))
    torch.cuda.synchronize()
    staged = len(stages) > 1
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)]
          for _ in range(steps)] if staged else None
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(s)
    for i in range(steps):
        a = args[i % copies]
        if staged:
            ev[i][0].record(s)
        for j, st in enumerate(stages):
            abi.check(st, fns[st](a, handle))
            if staged:
                ev[i][j + 1].record(s)
    stop.record(s)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    total_ms = start.elapsed_time(stop) / steps
    if not staged:
        return total_ms, wall, {}
    per_stage = {st: [] for st in stages}
    for i in range(steps):
        for j, st in enumerate(stages):
            per_stage[st].append(ev[i][j].elapsed_time(ev[i][j + 1]))
    return total_ms, wall, {k: (float(np.mean(v)), float(np.median(v)))
                            for k, v in per_stage.items()}


def device_warmup(tail, ms: float, copies: int) -> None:
    """Runs the step, untimed, for about `ms` of wall time (in batches of 64
    steps, synchronized) so that the timed steps run at steady-state clocks."""
    import torch
    from market_sim_amd import abi, ops
    if ms <= 0:
        return
    args = [tail.args(i % copies) for i in range(copies)]
    handle = tail.stream.cuda_stream
    t0 = time.perf_counter()
    i = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(64):
            abi.check("tail", ops.decode_tail_f16(args[i % copies], handle))
            i += 1
        torch.cuda.synchronize()


def back_to_back_ms(s, launch, launches: int) -> float:
    """Average ms of one launch among `launches` back-to-back launches on
    stream `s`, between two HIP events.  The launches are captured once into
    a HIP graph and the graph replayed, so that the host's per-call cost
    (a ctypes call per launch, more than a 10 us kernel) does not starve the
    GPU between launches; if capture is refused, an eager loop."""
    import torch
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    per = min(launches, 64)
    try:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(per):
                launch(i)
        reps = max(1, (launches + per - 1) // per)
        with torch.cuda.stream(s):  # a replay runs on the current stream
            g.replay()
            torch.cuda.synchronize()
            start.record(s)
            for _ in range(reps):
                g.replay()
            stop.record(s)
        torch.cuda.synchronize()
        ms = start.elapsed_time(stop) / (reps * per)
        del g
        return ms
    except RuntimeError:
        torch.cuda.synchronize()
    start.record(s)
    for i in range(launches):
        launch(i)
    stop.record(s)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / launches


def kernel_loop(tail, stage, launches, copies):
    """Average duration of one stage's kernel: back-to-back launches (rotating
    table copies) on the launch stream.  The stage must be idempotent given
    the prepare stage's outputs (both heads are: they read the normalized
    rows and write tile records)."""
    import torch
    from market_sim_amd import abi, ops
    fns = {"prepare": ops.decode_tail_prepare, "restricted": ops.decode_tail_restricted,
           "unrestricted": ops.decode_tail_unrestricted}
    args = [tail.args(i % copies) for i in range(copies)]
    s = tail.stream
    h = s.cuda_stream
    abi.check("prepare", ops.decode_tail_prepare(args[0], h))
    for i in range(10):
        abi.check(stage, fns[stage](args[i % copies], h))
    torch.cuda.synchronize()
    return back_to_back_ms(s, lambda i: abi.check(stage, fns[stage](args[i % copies], h)), launches)


def profiled_traffic(kernel: str, workload: str):
    """HBM-side bytes per launch of `kernel` on `workload` from that
    workload's committed rocprofv3 PMC summary (FETCH_SIZE and WRITE_SIZE
    passes scaled by a copy kernel of known size).  Returns (bytes, path of
    the summary), or (None, None) when no summary of this workload names the
    kernel."""
    rel = os.path.join("profiles", f"decode_tail_{workload}_traffic.md")
    try:
        for line in open(os.path.join(ROOT, rel)):
            if line.startswith("traffic_bytes_per_launch") and kernel in line:
                return int(line.split("=", 1)[1].split()[0]), rel
    except OSError:
        pass
    return None, None


def fallback_summary(alg: dict, fb_ms) -> dict:
    """The MFMA head's line on the gather path: its rows, launch time and
    roofline fractions; only when there are unrestricted rows (with none, the
    unrestricted stage launches nothing and a fraction would divide the head's
    bytes by an empty launch)."""
    if alg["B_u"] == 0 or fb_ms is None:
        return {"kernel": "none (no unrestricted rows)", "rows": 0}
    return {"kernel": "vocab_head_kernel (MFMA head, unrestricted rows)", "rows": alg["B_u"],
            "avg_launch_us": round(fb_ms * 1e3, 2),
            "hbm_GBs": round(alg["fallback_bytes"] / (fb_ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(alg["fallback_bytes"] / (fb_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "mfma_TFLOPs": round(alg["fallback_flops"] / (fb_ms * 1e-3) / 1e12, 2),
            "mfma_util": round(alg["fallback_flops"] / (fb_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}


def read_floor(tail, launches: int, copies: int) -> dict:
    """The same run's read floor: mf_read_floor over the rotated table copies
    (every byte once, 16-byte loads, contiguous chunks), `launches` back to
    back on the tail's stream."""
    import torch
    from market_sim_amd import abi, ops
    bufs = [ops.DeviceBuffer.of(t) for t in tail.tables[:copies]]
    sink_t = torch.zeros(4, dtype=torch.int32, device=tail.tables[0].device)
    sink = ops.DeviceBuffer.of(sink_t)
    s = tail.stream
    h = s.cuda_stream
    for i in range(10):
        abi.check("mf_read_floor", ops.read_floor(bufs[i % len(bufs)], sink, h))
    torch.cuda.synchronize()
    ms = back_to_back_ms(
        s, lambda i: abi.check("mf_read_floor", ops.read_floor(bufs[i % len(bufs)], sink, h)),
        launches)
    nbytes = bufs[0].size_bytes
    return {"kernel": "read_floor_kernel (mf_read_floor: the table, read once)",
            "bytes": nbytes, "avg_launch_us": round(ms * 1e3, 2),
            "GBs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def vendor_gemm(w, tail, launches: int) -> dict:
    """For scale beside the full-vocabulary comparator (which scores on this
    library's own MFMA projection kernel): the reference's full-path GEMM
    (linear.cu:92-102, FP16 inputs and logits) for the same shape, once as
    the vendor's torch.matmul on hipBLASLt and once as this library's
    mf_linear_f16 (the projection kernel), each timed back to back on the
    launch stream.  Both outputs are compared (FP16 logits, at most one ulp
    apart: FP32 accumulation in different orders)."""
    import torch
    from market_sim_amd import abi, ops
    dev = tail.tables[0].device
    g = torch.Generator(device="cpu").manual_seed(5)
    a = torch.randn(w.rows, w.hidden, generator=g).to(torch.float16).to(dev)
    e = tail.tables[0].view(torch.float16).reshape(w.vocab, w.hidden)
    out = torch.empty(w.rows, w.vocab, device=dev, dtype=torch.float16)
    own = torch.empty_like(out)
    s = tail.stream
    n = max(10, launches // 4)
    flops = 2.0 * w.rows * w.hidden * w.vocab

    def vendor_launch(_):
        torch.matmul(a, e.t(), out=out)

    args = (ops.DeviceBuffer.of(a).c(), ops.DeviceBuffer.of(e).c(), ops.DeviceBuffer.of(own).c(),
            w.rows, w.hidden, w.vocab, s.cuda_stream)

    def own_launch(_):
        abi.check("mf_linear_f16", abi.lib().mf_linear_f16(*args))

    with torch.cuda.stream(s):
        for _ in range(5):
            vendor_launch(0)
            own_launch(0)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        start.record(s)
        for _ in range(n):
            vendor_launch(0)
        stop.record(s)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / n
    own_ms = back_to_back_ms(s, own_launch, n)
    ob = own.view(torch.int16).to(torch.int32)
    vb = out.view(torch.int16).to(torch.int32)
    # FP16 patterns as integers adjacent for adjacent floats across zero
    ob = torch.where(ob < 0, -(ob & 0x7FFF), ob)
    vb = torch.where(vb < 0, -(vb & 0x7FFF), vb)
    max_ulps = int((ob - vb).abs().max().item())
    shape = f"[{w.rows}x{w.hidden}] x [{w.hidden}x{w.vocab}] -> FP16 logits"
    return {"op": f"torch.matmul FP16 {shape}", "ms": round(ms, 4),
            "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
            "projection_kernel": {"op": f"mf_linear_f16 {shape}", "ms": round(own_ms, 4),
                                  "TFLOPs": round(flops / (own_ms * 1e-3) / 1e12, 1),
                                  "max_ulps_vs_vendor": max_ulps}}


def cpu_baseline(w, budget_s: float) -> dict:
    """The CPU oracle (a plain-C port of the reference loops) on a bounded
    sample of the same pack: whole batches, all host threads, until the time
    budget is spent; plus one single-thread batch of a row subsample.

    The FP16 table is decoded to FP32 once, outside the timed region, as the
    reference's CPU model materializes FP32 weights
    (src/cpu/smollm2.cpp:65-174); the decoded values are exact, so the
    scores and tokens are the same bits as on the FP16 table."""
    import oracle

    # the box's CPU share (OMP_NUM_THREADS is set to it), else all cores
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    outputs = {}
    table = np.asarray(w.embedding)
    if table.dtype == np.uint16:
        table = table.view(np.float16).astype(np.float32)

    def one(threads_, rows=None):
        ww = w
        if rows is not None:
            import dataclasses
            ww = dataclasses.replace(w, x=w.x[rows], row_state=w.row_state[rows])
        t = time.perf_counter()
        out = oracle.decode_tail(ww.x, ww.norm_weight, ww.epsilon, table,
                                 ww.row_state, ww.state_offsets, ww.state_tokens,
                                 state_next=ww.state_next, next_table=ww.next_table,
                                 threads=threads_)
        if rows is None:
            outputs["full"] = out
        return time.perf_counter() - t, ww.rows

    one(threads)  # warm caches
    spent, seqs, reps = 0.0, 0, 0
    while spent < budget_s * 0.7 and reps < 20:
        dt, n = one(threads)
        spent += dt
        seqs += n
        reps += 1
    mt = seqs / spent
    # single thread on a 16-row slice (same restricted/unrestricted mix)
    rng = np.random.default_rng(0)
    rows = np.sort(rng.choice(w.rows, size=min(16, w.rows), replace=False))
    dt1, n1 = one(1, rows)
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(mt, 3), "unit": "seqs/s", "cores": threads, "kind": "port",
            "sample": f"{reps} full {w.name} batches ({seqs} sequences, "
                      f"{spent:.1f} s) of the oracle/oracle.c decode tail on "
                      f"{threads} threads, the FP16 table pre-decoded to FP32 "
                      f"outside the timed region; single thread {n1 / dt1:.3f} "
                      f"seqs/s on a {n1}-row slice",
            "table": "FP32, decoded from the FP16 table before timing",
            "single_thread_value": round(n1 / dt1, 3), "host_cpu": model,
            "_outputs": outputs["full"]}


def reference_bench() -> dict:
    """The reference's own restricted output-head benchmark (12 cells,
    src/tools/cuda_restricted_output_head_bench.cu) run by the C++ tool
    market_sim_amd/bench/restricted_output_head_bench in a child process;
    its document is checked against the reference schema and summarized
    next to the published L4 cells."""
    import subprocess
    from market_sim_amd import schema
    tool = os.path.join(ROOT, "market_sim_amd", "bench", "_build", "restricted_output_head_bench")
    if not os.path.exists(tool):
        return {"error": "tool not built (make -C market_sim_amd/bench)"}
    r = subprocess.run([tool], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        return {"error": f"exit {r.returncode}: {r.stderr.strip()[-300:]}"}
    doc = json.loads(r.stdout)
    schema.check_output_head_benchmark(doc)
    cells = schema.compare_with_l4(doc)
    ratios = [c["restricted_vs_l4"] for c in cells]
    return {
        "tool": "market_sim_amd/bench/restricted_output_head_bench",
        "gpu": doc["gpu"],
        "schema_ok": True,
        "token_parity_cells": sum(m["exact_token_parity"] for m in doc["measurements"]),
        "columns": ["rows", "allowed", "restricted_us", "full_us", "l4_restricted_us",
                    "l4_full_us"],
        "cells": [[c["rows"], c["allowed"], c["restricted_us"], c["full_us"],
                   c["l4_restricted_us"], c["l4_full_us"]] for c in cells],
        "restricted_vs_l4": [min(ratios), max(ratios)],
    }


def secondary_benches() -> dict:
    """The reference's restricted-greedy and RMSNorm benchmarks
    (src/tools/cuda_restricted_greedy_bench.cu, cuda_rmsnorm_bench.cu) run
    by the C++ tools market_sim_amd/bench/restricted_greedy_bench (on the
    market-action grammar of tests/golden/market_dfa.npz) and rmsnorm_bench
    with the reference's iteration counts; each document is checked against
    the reference schema and each tool checks its outputs (exit status)."""
    import subprocess
    import tempfile
    from market_sim_amd import schema
    from market_sim_amd.dfa import DfaTables, write_tables
    out = {}
    bdir = os.path.join(ROOT, "market_sim_amd", "bench", "_build")
    d = np.load(os.path.join(ROOT, "tests", "golden", "market_dfa.npz"))
    tables = DfaTables.from_arrays(d["offsets"], d["tokens"], d["next"], d["terminal"],
                                   vocab=49152)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "market.dfa")
        write_tables(tables, path)
        for name, cmd, check in (
                ("restricted_greedy", ["restricted_greedy_bench", "--dfa", path],
                 schema.check_restricted_greedy_benchmark),
                ("rms_norm", ["rmsnorm_bench"], schema.check_rmsnorm_benchmark)):
            tool = os.path.join(bdir, cmd[0])
            if not os.path.exists(tool):
                out[name] = {"error": "tool not built (make -C market_sim_amd/bench)"}
                continue
            r = subprocess.run([tool] + cmd[1:], capture_output=True, text=True, timeout=300)
            if r.returncode != 0:
                out[name] = {"error": f"exit {r.returncode}: {r.stderr.strip()[-300:]}"}
                continue
            doc = json.loads(r.stdout)
            check(doc)
            rate = "candidate_gib_per_second" if name == "restricted_greedy" \
                else "logical_gib_per_second"
            out[name] = {"checked": True, "columns": ["rows", "average_microseconds", rate],
                         "cells": [[m["rows"], m["average_microseconds"], m[rate]]
                                   for m in doc["measurements"]]}
            if name == "restricted_greedy":
                out[name]["seqs_per_s_at_256"] = doc["measurements"][-1]["sequences_per_second"]
    return out


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the path "
                          "shards by rows with no exchange",
                          "n_gpus": args.gpus}))
        return 2
    import torch
    from market_sim_amd import workloads
    from market_sim_amd.tail import DeviceTail

    w = workloads.config(args.config, seed=0)
    alg = algorithmic_bytes(w)
    tail = DeviceTail(w, copies=args.copies)
    # the clocks to their steady state first (untimed, reported)
    device_warmup(tail, args.device_warmup_ms, args.copies)
    # the step as a caller runs it: one mf_decode_tail_f16 call
    total_ms, wall_ms, _ = time_loop(tail, ["tail"], args.steps, args.warmup, args.copies)
    # per-kernel times: the four stage entry points, HIP events between them
    stages_ms, _, st = time_loop(tail, ["prepare", "restricted", "unrestricted", "finalize"],
                                 args.steps, max(5, args.warmup // 2), args.copies)
    # correctness of what was timed: the last step's outputs vs the oracle on
    # a row sample is checked in tests; here record a token checksum
    tok, sc, nx = tail.results()
    if args.calibration_copy_mib:
        n = args.calibration_copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        del src, dst
    # the dominant kernel: the one-kernel tail (short lists, no unrestricted
    # rows: the prepare stage is the whole step), the table pass (sorted
    # lists with unrestricted rows: one kernel for both kinds of rows) or
    # the CSR gather
    one_pass = tail.table_pass
    fused = tail.fused
    dense = tail.dense
    main_ms = kernel_loop(tail, "prepare" if fused else ("unrestricted" if dense else "restricted"),
                          args.steps, args.copies)
    if dense:
        # the dense head (unrestricted rows and long ascending lists, one pass
        # over the table) dominates; the gather takes the other rows
        main_bytes = alg["dense_bytes"]
        main_name = "dense_kernel (dense head: unrestricted rows + long ascending lists)"
        achieved = main_bytes / (main_ms * 1e-3) / 1e9
        traffic, traffic_source = profiled_traffic("dense_kernel", w.name)
        rest_ms = kernel_loop(tail, "restricted", args.steps, args.copies)
        fb = {"kernel": "inside dense_kernel (MFMA on the FP16 hi of z)",
              "rows": alg["B_u"], "dense_list_rows": alg["D"],
              "mfma_TFLOPs": round(alg["dense_flops"] / (main_ms * 1e-3) / 1e12, 2),
              "mfma_util": round(alg["dense_flops"] / (main_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
              "gather_rest": {"kernel": "gather_mfma_kernel (the other restricted rows)",
                              "rows": alg["B_rest"], "avg_launch_us": round(rest_ms * 1e3, 2),
                              "hbm_frac": round(alg["gather_rest"] / (rest_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                              "logical_frac": round(alg["gather_rest_logical"] / (rest_ms * 1e-3) / 1e9 /
                                                    HBM_PEAK_GBS, 4)}}
    elif fused:
        # the same bytes as the gather: each distinct candidate row, the ids,
        # the hidden rows, the offsets and the outputs
        main_bytes = alg["gather"]
        main_name = "short_tail_kernel (one kernel: norm, exact scores, selection, DFA advance)"
        achieved = main_bytes / (main_ms * 1e-3) / 1e9
        traffic, traffic_source = profiled_traffic("short_tail_kernel", w.name)
        fb = {"kernel": "none (no unrestricted rows)", "rows": alg["B_u"]}
    elif one_pass:
        main_bytes, main_name = alg["pass_bytes"], "pass_kernel (one table pass: candidates + unrestricted head)"
        achieved = main_bytes / (main_ms * 1e-3) / 1e9
        traffic, traffic_source = profiled_traffic("pass_kernel", w.name)
        fb = {"kernel": "inside pass_kernel (MFMA on the FP16 hi of z)", "rows": alg["B_u"],
              "mfma_TFLOPs": round(alg["pass_flops"] / (main_ms * 1e-3) / 1e12, 2),
              "mfma_util": round(alg["pass_flops"] / (main_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
    else:
        main_bytes, main_name = alg["gather"], "gather_mfma_kernel (CSR gather)"
        achieved = main_bytes / (main_ms * 1e-3) / 1e9
        traffic, traffic_source = profiled_traffic("gather_mfma_kernel", w.name)
        fb_ms = kernel_loop(tail, "unrestricted", args.steps, args.copies) if alg["B_u"] > 0 else None
        fb = fallback_summary(alg, fb_ms)
    floor = read_floor(tail, args.steps, args.copies)
    result = {
        "metric": METRIC,
        "value": round(w.rows / (total_ms * 1e-3), 1),
        "unit": "seqs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "device_warmup_ms": args.device_warmup_ms,
        "ms_per_step": round(total_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded PCG64; N(0,0.02) FP16 table, N(0,1) hidden)",
        "config": {"workload": w.name, "rows": w.rows, "hidden": w.hidden,
                   "vocab": w.vocab, "sizes": w.sizes,
                   "unrestricted_rows": alg["B_u"], "candidates": alg["N"],
                   "distinct_ids": alg["U"], "table_copies": args.copies,
                   "order": "fma chain (greedy.cu:171-176)"},
        "roofline": {"kernel": main_name, "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": main_bytes, "avg_launch_us": round(main_ms * 1e3, 2),
                     "traffic_source": traffic_source},
        "stages_us": {k: round(v[0] * 1e3, 2) for k, v in st.items()},
        "stages_serial_ms": round(stages_ms, 5),
        "effective_gather_GBs": round(alg["gather_logical"] / (main_ms * 1e-3) / 1e9, 1),
        "fallback": fb,
        "read_floor": floor,
        "wall_ms_per_step": round(wall_ms, 4),
        "token_checksum": int(np.bitwise_xor.reduce(tok.astype(np.uint64) * np.arange(1, tok.size + 1, dtype=np.uint64))),
    }
    if one_pass:
        # the table pass against a plain read of the same table
        result["roofline"]["vs_read_floor"] = round(floor["avg_launch_us"] / (main_ms * 1e3), 4)
    if one_pass and not args.no_gather_path:
        # the same step on the gather + MFMA head kernels (no sorted-lists
        # declaration), same tokens required
        g = DeviceTail(w, copies=args.copies, sorted_lists=False)
        g_ms, _, _ = time_loop(g, ["tail"], args.steps, args.warmup, args.copies)
        gtok, _, _ = g.results()
        g_gather = kernel_loop(g, "restricted", args.steps, args.copies)
        g_head = kernel_loop(g, "unrestricted", args.steps, args.copies) if alg["B_u"] > 0 else None
        head = fallback_summary(alg, g_head)
        result["gather_path"] = {
            "ms_per_step": round(g_ms, 5), "token_parity": bool(np.array_equal(gtok, tok)),
            "gather_us": round(g_gather * 1e3, 2),
            "gather_frac": round(alg["gather"] / (g_gather * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if g_head is not None:
            result["gather_path"]["head_us"] = head["avg_launch_us"]
            result["gather_path"]["head_frac"] = head["hbm_frac"]
        del g
    if dense and not args.no_gather_path:
        # the same step with every restricted row on the gather and the MFMA
        # head for the unrestricted rows (MF_TAIL_NO_DENSE), same tokens
        # required
        g = DeviceTail(w, copies=args.copies, dense=False)
        g_ms, _, _ = time_loop(g, ["tail"], args.steps, args.warmup, args.copies)
        gtok, _, _ = g.results()
        g_gather = kernel_loop(g, "restricted", args.steps, args.copies)
        g_head = kernel_loop(g, "unrestricted", args.steps, args.copies) if alg["B_u"] > 0 else None
        result["gather_path"] = {
            "ms_per_step": round(g_ms, 5), "token_parity": bool(np.array_equal(gtok, tok)),
            "gather_us": round(g_gather * 1e3, 2),
            "gather_frac": round(alg["gather"] / (g_gather * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if g_head is not None:
            result["gather_path"]["head_us"] = round(g_head * 1e3, 2)
        del g
    if fused and not args.no_gather_path:
        # the same step on the separate kernels (MF_TAIL_NO_FUSED)
        g = DeviceTail(w, copies=args.copies, fused=False)
        g_ms, _, _ = time_loop(g, ["tail"], args.steps, args.warmup, args.copies)
        gtok, _, _ = g.results()
        result["separate_kernels"] = {"ms_per_step": round(g_ms, 5),
                                      "token_parity": bool(np.array_equal(gtok, tok))}
        del g
    if not args.no_full:
        full = DeviceTail(w, copies=args.copies, full=True)
        full_ms, _, _ = time_loop(full, ["full"], max(10, args.steps // 4), 5, args.copies)
        ftok, _, _ = full.results()
        result["vs_full_head"] = round(full_ms / total_ms, 3)
        result["full_head_ms"] = round(full_ms, 4)
        result["full_head_token_parity"] = bool(np.array_equal(ftok, tok))
        del full
        result["vendor_gemm"] = vendor_gemm(w, tail, args.steps)
        result["vs_vendor_gemm"] = round(result["vendor_gemm"]["ms"] / total_ms, 3)
    if not args.no_reference_bench:
        result["reference_bench"] = reference_bench()
        result["secondary_benches"] = secondary_benches()
    if not args.no_cpu:
        cb = cpu_baseline(w, args.cpu_seconds)
        etok, esc, enx = cb.pop("_outputs")
        result["cpu_baseline"] = cb
        result["vs_cpu"] = round(result["value"] / cb["value"], 1)
        # the timed GPU outputs against the oracle on the same inputs
        nan = np.isnan(esc)
        result["parity"] = {
            "tokens_bit_exact": bool(np.array_equal(tok, etok)),
            "scores_bit_exact": bool(np.array_equal(np.isnan(sc), nan) and np.array_equal(
                sc[~nan].view(np.uint32), esc[~nan].view(np.uint32))),
            "next_states_bit_exact": bool(np.array_equal(nx, enx)),
        }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
