"""Benchmark of the W4A16 fused dequant-GEMM on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--sweep]
    python bench.py --reference-table [--reference-json PATH]

Prints ONE JSON line.  Headline (``value``): HBM GB/s of the decode GEMV at
BASELINE config C2 (M=1, K=N=4096, G=128) -- algorithmic bytes per call
(2MK + 4(K/8)N + 4(K/G)N + 2MN, reference bench_gemm.py:61-67) over the average
time per call.  Timing of the K steps:

* weights cold: the calls cycle over enough copies of (qweight, scales, zeros)
  that they total > 512 MiB, and right before the timed calls one untimed call
  reads every copy in order, so the copy each timed call reads was last read
  (copies) calls -- more than 512 MiB of other weights -- earlier: the 256 MiB
  Infinity Cache cannot hold it, at any K;
* the W warm-up calls, the rotation and the K timed calls are eager launches
  on one stream, all queued behind a bounded spin kernel (torch.cuda._sleep)
  so the host has issued every one before the GPU starts: the GPU runs them
  back to back, busy up to the timed calls, and the figure holds neither the
  host's launch cost (~12 us per Python call) nor a graph launch.  HIP events
  on that stream bracket exactly the K calls; ``ms_per_step`` = event time / K;
* ``secondary``: TFLOP/s of the prefill MFMA GEMM at C4 M=4096 (2MNK flops),
  its calls timed as one HIP-graph replay (SECONDARY_GRAPH says why) after
  enough untimed calls for the clock to settle under this load;
* ``cpu_baseline``: the CPU oracle's dequantise-then-matmul path
  (``oracle/w4a16_oracle.reference_w4a16``, a numpy port of the reference's
  reference.py:18-40) on the same C2 inputs, on every host core the process may
  use (columns split over threads: GEMM columns are independent), over a
  bounded number of calls.

``--reference-table`` instead reproduces the reference's own benchmark
(w4a16-kernel/benchmarks/bench_gemm.py): its method (warm weights, eager
calls, 25 warm-up calls, median of 100 calls each bracketed by events and a
synchronize), its result keys (fp16_ms, dequant_matmul_ms, w4a16_ms, ...,
speedup_vs_fp16, speedup_vs_dequant) and its markdown table, over its
DEFAULT_SHAPES and the BASELINE configurations' shapes.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "w4a16-dequant-fused-matmul-kernel_amd")
for _p in (ROOT, PKG_DIR):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP16_PEAK_TFLOPS = 2516.6      # MI355X dense fp16 MFMA
COLD_BYTES = 512 << 20
SPIN_CYCLES_PER_US = 2500      # the spin kernel counts shader clocks (<= 2.4 GHz)
# The prefill line runs as one graph replay: its kernels run ~6 % faster inside a
# graph than as separate eager dispatches (kernel trace, C4 M=4096: median 400.6
# vs 421.7 us), and at ~0.4 ms per call the replay's launch (~9 us) is 0.5 % of
# 50 calls.  The decode headline runs eager: there the graph's launch would be
# 0.45 us of a ~5 us call at K = 20.
SECONDARY_GRAPH = True


def _args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-secondary", action="store_true", help="skip the C4 prefill line")
    ap.add_argument("--sweep", action="store_true",
                    help="also time every C2-C5 case (stderr table, --sweep-json file)")
    ap.add_argument("--sweep-json", default=None)
    ap.add_argument("--graph", action="store_true",
                    help="time one HIP-graph replay of the K calls instead of eager calls "
                         "(includes the graph's launch latency)")
    ap.add_argument("--reference-table", action="store_true",
                    help="the reference's bench_gemm.py method, keys and markdown table")
    ap.add_argument("--reference-json", default=None, help="write the --reference-table rows here")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run the workloads for rocprofv3 --pmc: a 256 MiB copy "
                         "(calibration), then cold C2 decode calls, C3 small-batch calls "
                         "(skinny and 32-row streamed kernels) and C4 M=4096 prefill "
                         "calls (PROBE); no timing")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write profiles/traffic.json from the counter_collection.csv files "
                         "of two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of "
                         "--traffic-probe")
    ap.add_argument("--empty-kernels", action="store_true",
                    help="time K calls of two near-empty kernels exactly as the headline's "
                         "calls are timed (eager, behind the spin, HIP events): the per-dispatch "
                         "cost of the queue itself, untraced or under a tracer")
    ap.add_argument("--planner-audit", action="store_true",
                    help="planner regret: the static plan against every other plan the "
                         "library has (w4a16.autotune.candidates) over LLM layer shapes x M "
                         "(AUDIT_SHAPES, AUDIT_MS); markdown table")
    ap.add_argument("--audit-shapes", default=None,
                    help="comma list of KxN (default: AUDIT_SHAPES)")
    ap.add_argument("--audit-ms", default=None, help="comma list of M (default: AUDIT_MS)")
    ap.add_argument("--audit-g", type=int, default=128, help="group size of the audit (default 128)")
    ap.add_argument("--decode-scan", metavar="OUT_JSON",
                    help="time every GEMV and skinny plan for M = 1, 2 (G = --audit-g) over "
                         "the DECODE_KS x DECODE_NS grid, cold weights; JSON for --decode-table")
    ap.add_argument("--decode-ks", default=None,
                    help="with --decode-scan: comma list of K (default: DECODE_KS)")
    ap.add_argument("--decode-ns", default=None,
                    help="with --decode-scan: comma list of N (default: DECODE_NS)")
    ap.add_argument("--decode-table", metavar="SCAN_JSON", nargs="+",
                    help="write csrc/decode_table.inc (the planner's measured M <= 2 table) "
                         "from --decode-scan files (group-size classes they do not cover keep "
                         "their current entries; a later file's shapes replace an earlier's)")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="markdown table of a rocprofv3 --kernel-trace CSV of bench.py: per "
                         "kernel, the durations of its last --steps dispatches (the timed "
                         "calls) and the gaps between them")
    ap.add_argument("--trace-last", default=None, metavar="NAME=COUNT,...",
                    help="with --trace-summary: timed-call counts for kernels whose names "
                         "contain NAME (default --steps for all)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="CSV",
                    help="markdown table of every counter in rocprofv3 --pmc runs of "
                         "--traffic-probe, per workload and kernel")
    return ap.parse_args()


def _time_calls(fns, steps: int, warmup: int, graph: bool) -> dict:
    """Average ms per call of `fns` (call i runs fns[i % len(fns)]), HIP events
    on the stream the kernels run on.

    In order on one stream: W warm-up calls, one call on every element of
    `fns` in order (the rotation that leaves the timed calls' weights cold),
    then the K timed calls between two events.  All of it is queued behind one
    spin kernel, sized from the host's measured launch rate, so the GPU runs
    warm-up, rotation and timed calls back to back -- busy (and clocked up)
    right to the start event -- and none waits on the host; if the GPU reached
    the start event before the host had queued everything, the whole sequence
    runs again behind a longer spin.  Eager (default): the K calls are K
    launches.  Graph: they are one graph, replayed once untimed beforehand."""
    import torch

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        fns[0]()                             # first call: plan, workspace, code load
        stream.synchronize()
        t0 = time.perf_counter()
        for f in fns:                        # untimed: the host's launch rate
            f()
        host_us = (time.perf_counter() - t0) / len(fns) * 1e6
    stream.synchronize()
    g = None
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(steps):
                fns[i % len(fns)]()
        with torch.cuda.stream(stream):
            g.replay()                      # untimed: uploads the graph
        stream.synchronize()
    n_queued = warmup + len(fns) + (1 if graph else steps)
    for attempt in range(4):
        spin_us = (200 + 2 * host_us * n_queued) * 4 ** attempt
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            torch.cuda._sleep(int(SPIN_CYCLES_PER_US * spin_us))
            for i in range(warmup):
                fns[i % len(fns)]()
            for f in fns:                        # rotation: every copy, in order
                f()
            start.record(stream)
            if graph:
                g.replay()
            else:
                for i in range(steps):
                    fns[i % len(fns)]()
            end.record(stream)
            # the GPU must not have reached the start event before every call
            # was queued, or the timed calls would have waited on the host
            queued = not start.query()
        end.synchronize()
        torch.cuda.synchronize()
        if queued:
            break
    return {"ms": start.elapsed_time(end) / steps, "queued_before_start": queued,
            "host_us_per_call": host_us, "spin_us": spin_us}


def empty_kernels(steps: int, warmup: int) -> dict:
    """Per-call time of near-empty kernels queued and timed like the headline's
    calls: torch.cuda._sleep(0) (one thread, no work) and a fill of 128 Ki fp16
    (torch's elementwise kernel over a grid of workgroups).  What the queue
    costs per dispatch; run under rocprofv3 --kernel-trace as well, it shows
    what the tracer adds to each dispatch."""
    import torch

    buf = torch.empty(256 * 512, dtype=torch.float16, device="cuda")
    out = {}
    for name, fn in (("sleep0", lambda: torch.cuda._sleep(0)), ("fill_128Ki_f16", lambda: buf.fill_(1.0))):
        t = _time_calls([fn], steps, warmup, False)
        out[name] = {"us_per_call": round(t["ms"] * 1e3, 4),
                     "queued_before_start": t["queued_before_start"]}
    return {"what": "near-empty kernels, K eager calls behind a spin kernel, HIP events",
            "steps": steps, "warmup": warmup, "kernels": out}


def trace_summary(path: str, last: int, per_kernel: str | None = None) -> str:
    """Markdown table from a rocprofv3 kernel-trace CSV: per kernel, the
    number of dispatches, and over its last `last` dispatches (bench.py's timed
    calls are each kernel's last ones) the mean / median / min / max duration,
    the mean gap from one dispatch's end to the next one's start, and the span
    from the first one's start to the last one's end per dispatch (what HIP
    events around those calls measure).  `per_kernel` ("name=count,...")
    gives kernels whose names contain `name` another count (the prefill line
    times 50 calls: "stream_kernel=50,Cijk=50")."""
    import csv
    import statistics

    by = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            by.setdefault(r["Kernel_Name"], []).append(
                (int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    counts = {}
    for item in (per_kernel or "").split(","):
        if "=" in item:
            k, v = item.split("=")
            counts[k.strip()] = int(v)
    lines = ["| kernel | dispatches | timed (last) | mean ns | median ns | min ns | max ns | "
             "mean gap ns | span / dispatch ns |", "|---|---|---|---|---|---|---|---|---|"]
    for name, ds in sorted(by.items(), key=lambda kv: -len(kv[1])):
        ds.sort()
        n = next((v for k, v in counts.items() if k in name), last)
        tail = ds[-n:]
        dur = [e - s for s, e in tail]
        gaps = [tail[i + 1][0] - tail[i][1] for i in range(len(tail) - 1)]
        gap = f"{statistics.mean(gaps):.0f}" if gaps else ""
        span = (tail[-1][1] - tail[0][0]) / len(tail)
        lines.append(f"| `{_kernel_short(name)}` | {len(ds)} | {len(tail)} | "
                     f"{statistics.mean(dur):.0f} | {statistics.median(dur):.0f} | {min(dur)} | "
                     f"{max(dur)} | {gap} | {span:.0f} |")
    return "\n".join(lines)


def _layer_copies(qw, sc, zr, n: int) -> list:
    """`n` copies of one quantised layer (the first the tensors themselves where
    their scales and zeros already lie close together), each copy's scales and
    zeros the two halves of one allocation.  The streamed prefill kernels read
    scales and zeros through one buffer resource and need them within 2 GiB
    of each other (further apart the library runs its register-tiled kernel
    instead); separate allocations in a process that has allocated and freed
    many large tensors do not guarantee that, and a timing should measure the
    planned kernel."""
    import torch
    from w4a16.hip_kernel import mark_integer_zeros

    def packed(q):
        sz = torch.empty((2,) + tuple(sc.shape), dtype=sc.dtype, device=sc.device)
        sz[0].copy_(sc)
        sz[1].copy_(zr)
        mark_integer_zeros(sz[1])
        return q, sz[0], sz[1]

    near = abs(sc.data_ptr() - zr.data_ptr()) + sc.numel() * 2 < (1 << 30)
    first = (qw, sc, zr) if near else packed(qw)
    return [first] + [packed(qw.clone()) for _ in range(n - 1)]


def _prepare(case, copies_for_cold: bool):
    import torch
    from w4a16 import quantize_weight
    from w4a16 import workloads as wl

    X, W = wl.make_inputs(case)
    Xd = X.cuda()
    qw, s, z = quantize_weight(W.cuda(), case.G)
    per_copy = qw.numel() * 4 + s.numel() * 2 + z.numel() * 2
    ncopy = 1
    if copies_for_cold:
        ncopy = max(2, -(-COLD_BYTES // per_copy) + 1)
    layers = _layer_copies(qw, s, z, ncopy)
    y = torch.empty(case.M, case.N, dtype=torch.float16, device="cuda")
    return X, W, Xd, layers, y, ncopy, per_copy


def bench_case(case, steps: int, warmup: int, graph: bool = False, cold: bool = True) -> dict:
    from w4a16 import w4a16_matmul
    from w4a16.hip_kernel import plan_for

    X, W, Xd, layers, y, ncopy, per_copy = _prepare(case, cold)
    fns = [(lambda l=l: w4a16_matmul(Xd, l[0], l[1], l[2], case.G, out=y)) for l in layers]
    t = _time_calls(fns, steps, warmup, graph)
    ms = t["ms"]
    p = plan_for(case.M, case.N, case.K, case.G).as_dict()
    us = ms * 1e3
    gbs = case.bytes() / (ms * 1e-3) / 1e9
    tflops = case.flops() / (ms * 1e-3) / 1e12
    return {"case": case.name, "M": case.M, "K": case.K, "N": case.N, "G": case.G,
            "steps": steps, "us": us, "GB/s": gbs, "TFLOP/s": tflops, "weight_copies": ncopy,
            "copy_mib": per_copy / 2**20, "queued_before_start": t["queued_before_start"],
            "graph": graph, "host_us_per_call": round(t["host_us_per_call"], 1),
            "kernel": p["kernel_name"], "split_k": p["split_k"], "tile_cfg": p["tile_cfg"],
            "tile": [p["tile_m"], p["tile_n"]], "grid": [p["grid_x"], p["grid_y"]],
            "bytes": case.bytes(), "flops": case.flops()}


def dense_fp16_case(case, steps: int, warmup: int) -> dict:
    """Context for the prefill line: torch's fp16 GEMM (hipBLASLt) of the same
    M x K x N with an fp16 W (4x the weight bytes, no dequant), timed the same
    way (one graph replay of the calls, HIP events) right after it."""
    import torch
    from w4a16 import workloads as wl

    X, W = (t.cuda() for t in wl.make_inputs(case))
    y = torch.empty(case.M, case.N, dtype=torch.float16, device="cuda")
    t = _time_calls([lambda: torch.matmul(X, W, out=y)], steps, warmup, True)
    us = t["ms"] * 1e3
    return {"what": "torch.matmul fp16 x fp16 (hipBLASLt), same shape and timing",
            "us": round(us, 2), "TFLOP/s": round(case.flops() / us / 1e6, 2)}


def bench_quantize(case, steps: int, warmup: int) -> dict:
    """quantize_weight's kernel (w4a16_quantize_pack_f16) on the case's fp16 W,
    outputs preallocated, calls queued behind the spin and timed with HIP
    events like the GEMM cases; GB/s of W read plus qweight, scales and zeros
    written.  W (K x N fp16) is far larger than the caches only at C4 / C5
    sizes; at C2 (32 MiB) consecutive calls may find part of it in the 256 MiB
    Infinity Cache."""
    import torch
    from w4a16 import _lib
    from w4a16 import workloads as wl

    _, W = wl.make_inputs(case)
    Wd = W.cuda()
    K, N, G = case.K, case.N, case.G
    qw = torch.empty(K // 8, N, dtype=torch.int32, device="cuda")
    sc = torch.empty(K // G, N, dtype=torch.float16, device="cuda")
    zr = torch.empty(K // G, N, dtype=torch.float16, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    lib = _lib.load()

    def call():
        rc = lib.w4a16_quantize_pack_f16(Wd.data_ptr(), qw.data_ptr(), sc.data_ptr(),
                                         zr.data_ptr(), K, N, G, flag.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream)
        if rc:
            raise RuntimeError(f"w4a16_quantize_pack_f16: {rc}")
    t = _time_calls([call], steps, warmup, False)
    nbytes = 2 * K * N + 4 * (K // 8) * N + 2 * 2 * (K // G) * N
    us = t["ms"] * 1e3
    return {"case": "quantize " + case.name, "K": K, "N": N, "G": G, "us": us,
            "GB/s": nbytes / us / 1e3, "bytes": nbytes, "flag": int(flag.item())}


# --planner-audit: (label, K, N) of Llama-style layers: fused QKV, out-proj,
# fused gate+up, down-proj of 7B (Llama-2), 8B (Llama-3), 13B and 70B.
AUDIT_SHAPES = [("7B qkv", 4096, 12288), ("7B o", 4096, 4096), ("7B gate+up", 4096, 22016),
                ("7B down", 11008, 4096), ("8B qkv", 4096, 6144), ("8B gate+up", 4096, 28672),
                ("8B down", 14336, 4096), ("13B qkv", 5120, 15360), ("13B o", 5120, 5120),
                ("13B gate+up", 5120, 27648), ("13B down", 13824, 5120),
                ("70B qkv", 8192, 10240), ("70B o", 8192, 8192), ("70B gate+up", 8192, 57344),
                ("70B down", 28672, 8192)]
AUDIT_MS = [1, 2, 4, 8, 16, 32, 64, 96, 128, 192, 256, 512, 1024]


def planner_audit(shapes, ms, G: int = 128, steps: int = 30, reps: int = 3) -> str:
    """Markdown table: per shape and M, the static plan's µs against the fastest
    of the other plans (timed the bench's way: cold weights and eager calls for
    M < 64, warm weights in a graph replay from M = 64; repetitions interleaved
    across plans; median).  The static plan is timed twice (its two medians
    give the run's noise).  Regret = static / best - 1."""
    import torch
    from w4a16 import autotune, quantize_weight
    from w4a16.hip_kernel import w4a16_matmul_planned

    lines = ["| layer | K | N | M | static plan | static µs | static µs (again) | best plan | "
             "best µs | regret |", "|---|---|---|---|---|---|---|---|---|---|"]
    worst = []
    for label, K, N in shapes:
        g = torch.Generator(device="cuda").manual_seed(K * 7 + N)
        W = (torch.randn(K, N, device="cuda", generator=g) * 0.02).to(torch.float16)
        qw, sc, zr = quantize_weight(W, G)
        del W
        per = qw.numel() * 4 + sc.numel() * 4
        for M in ms:
            X = torch.randn(M, K, device="cuda", generator=g).to(torch.float16)
            cold = M < 64
            ncopy = max(2, -(-COLD_BYTES // per) + 1) if cold else 1
            layers = _layer_copies(qw, sc, zr, ncopy)
            y = torch.empty(M, N, dtype=torch.float16, device="cuda")
            cands = autotune.candidates(M, N, K, G)
            cands = [cands[0], ("static (again)", cands[0][1])] + cands[1:]
            live = []
            for name, p in cands:
                try:
                    w4a16_matmul_planned(X, qw, sc, zr, G, p, out=y)
                except RuntimeError:
                    continue
                fns = [(lambda l=l, p=p: w4a16_matmul_planned(X, l[0], l[1], l[2], G, p, out=y))
                       for l in layers]
                live.append((name, fns))
            torch.cuda.synchronize()
            times = {name: [] for name, _ in live}
            best_first = float("inf")
            for r in range(reps):
                for name, fns in live:
                    if r > 0 and times[name][0] > 1.5 * best_first and not name.startswith("static"):
                        continue
                    t = _time_calls(fns, steps, 5, not cold)["ms"] * 1e3
                    times[name].append(t)
                    if r == 0:
                        best_first = min(best_first, t)
            import statistics
            med = {n: statistics.median(v) for n, v in times.items()}
            st, st2 = med[cands[0][0]], med["static (again)"]
            others = {n: v for n, v in med.items() if not n.startswith("static")}
            bname = min(others, key=others.get) if others else cands[0][0]
            best = min(others.get(bname, st), st, st2)
            if best >= min(st, st2):
                bname = "static"
            regret = st / best - 1.0
            worst.append((regret, label, M, bname))
            lines.append(f"| {label} | {K} | {N} | {M} | {cands[0][1].as_dict()['kernel_name']} "
                         f"cfg {cands[0][1].tile_cfg} split {cands[0][1].split_k} "
                         f"tile {cands[0][1].tile_m}x{cands[0][1].tile_n} | {st:.2f} | {st2:.2f} | "
                         f"{bname} | {best:.2f} | {100 * regret:+.1f} % |")
            print(lines[-1], file=sys.stderr, flush=True)
            del layers, X, y
        del qw, sc, zr
        torch.cuda.empty_cache()
    worst.sort(reverse=True)
    n3 = sum(1 for w in worst if w[0] > 0.03)
    lines.append("")
    lines.append(f"{len(worst)} shapes x M; static plan more than 3 % behind the best other plan "
                 f"on {n3}; largest regrets: " +
                 "; ".join(f"{l} M={m} {100 * r:+.1f} % ({b})" for r, l, m, b in worst[:5]))
    return "\n".join(lines)


# --decode-scan grid: the planner's measured table for M <= 2, G % 128 == 0
# covers K in [DECODE_KS[0], DECODE_KS[-1]] and N in [DECODE_NS[0], DECODE_NS[-1]]
DECODE_KS = [3584, 4096, 5120, 6144, 8192, 11008, 13824, 14336, 16384, 20480, 28672]
DECODE_NS = [4096, 5120, 6144, 8192, 10240, 11008, 12288, 14336, 15360, 16384, 20480, 22016,
             24576, 27648, 28672, 32768, 40960, 57344, 65536, 98304, 131072, 163840]
DECODE_TABLE = os.path.join(PKG_DIR, "csrc", "decode_table.inc")


def decode_scan(out_path: str, ks=None, ns=None, ms=(1, 2), G: int = 128) -> None:
    """Median µs of every GEMV and skinny plan (w4a16.autotune.candidates) at each
    (M, K, N) of the grid, timed the bench's way (cold weights, eager calls
    behind the spin, 3 interleaved repetitions); written as JSON after every
    (K, N)."""
    import statistics

    import torch
    from w4a16 import _lib, autotune, quantize_weight
    from w4a16.hip_kernel import w4a16_matmul_planned

    res = []
    for K in ks or DECODE_KS:
        for N in ns or DECODE_NS:
            g = torch.Generator(device="cuda").manual_seed(K + N)
            W = (torch.randn(K, N, device="cuda", generator=g) * 0.02).to(torch.float16)
            qw, sc, zr = quantize_weight(W, G)
            del W
            per = qw.numel() * 4 + sc.numel() * 4
            ncopy = max(2, -(-COLD_BYTES // per) + 1)
            layers = _layer_copies(qw, sc, zr, ncopy)
            for M in ms:
                X = torch.randn(M, K, device="cuda", generator=g).to(torch.float16)
                y = torch.empty(M, N, dtype=torch.float16, device="cuda")
                live = []
                for name, p in autotune.candidates(M, N, K, G):
                    if name != "static" and p.kernel not in (_lib.KERNEL_GEMV, _lib.KERNEL_SKINNY):
                        continue
                    try:
                        w4a16_matmul_planned(X, qw, sc, zr, G, p, out=y)
                    except RuntimeError:
                        continue
                    fns = [(lambda l=l, p=p: w4a16_matmul_planned(X, l[0], l[1], l[2], G, p,
                                                                  out=y)) for l in layers]
                    live.append((name, p, fns))
                t = {name: [] for name, _, _ in live}
                for _ in range(3):
                    for name, p, fns in live:
                        t[name].append(_time_calls(fns, 30, 5, False)["ms"] * 1e3)
                res.append({"M": M, "K": K, "N": N, "G": G,
                            "plans": {name: p.as_dict() for name, p, _ in live},
                            "us": {name: statistics.median(v) for name, v in t.items()}})
                best = min(res[-1]["us"], key=res[-1]["us"].get)
                print(f"M={M} K={K} N={N} static {res[-1]['us']['static']:.2f} best {best} "
                      f"{res[-1]['us'][best]:.2f}", file=sys.stderr, flush=True)
                del X, y
            del layers, qw, sc, zr
            torch.cuda.empty_cache()
            with open(out_path, "w") as f:
                json.dump(res, f)


def decode_table(scan_paths) -> str:
    """C source of the planner's M <= 2 table from --decode-scan files: per
    group-size class (128: G % 128 == 0, 64: G % 64 == 0, 32: other G % 32 == 0)
    and measured (M, K, N) the fastest plan (family, configuration, column
    block or row group, k-split).  Classes the files do not cover keep the
    entries the current table holds for them; where files measure the same
    shape, the later file's measurement is taken."""
    def gclass(G: int) -> int:
        return 128 if G % 128 == 0 else 64 if G % 64 == 0 else 32

    rows = []
    for path in scan_paths:
        with open(path) as f:
            rows += json.load(f)
    scanned = {gclass(r.get("G", 128)) for r in rows}
    kept = []
    if os.path.exists(DECODE_TABLE):
        for ln in open(DECODE_TABLE).read().splitlines():
            if ln.startswith("{") and int(ln[1:].split(",")[0]) not in scanned:
                kept.append(ln)
    lines = ["// Generated by `python bench.py --decode-table <scan.json> ...` from",
             "// `python bench.py --decode-scan <scan.json> [--audit-g G]` on one MI355X",
             "// (256 CUs): per group-size class (128: G % 128 == 0, 64: G % 64 == 0,",
             "// 32: other G % 32 == 0) and (M, K, N) of the grid, cold weights, the",
             "// fastest GEMV / skinny plan.  Fields: G class, M, K, N, kernel (1 GEMV,",
             "// 4 skinny), tile_cfg, tile_n, tile_m (skinny rows), split_k, µs x 100 of",
             "// the fastest, of the plan the planner gave when scanned (0: the grid",
             "// point's weights exceed the vector kernels' 2 GiB limit; the entry repeats",
             "// the nearest fitting K's plan for the fitting shapes around it).",
             "// clang-format off"]
    latest = {}
    for r in rows:
        latest[(gclass(r.get("G", 128)), r["M"], r["K"], r["N"])] = r

    def fastest(r):
        us = r["us"]
        best = min(us, key=us.get)
        return best, r["plans"][best]

    new = []
    for key, r in latest.items():
        best, p = fastest(r)
        us = r["us"]
        b_us, s_us = round(100 * us[best]), round(100 * us["static"])
        if p["kernel"] not in (1, 4):
            # the grid point's operands exceed the vector kernels' 2 GiB
            # limit (only the SIMT plan ran): repeat the plan of the nearest
            # K that fits, for the fitting shapes around the point, and mark
            # the entry with 0 us
            near = [v for k, v in latest.items() if k[:2] == key[:2] and k[3] == key[3]
                    and fastest(v)[1]["kernel"] in (1, 4)]
            if near:
                p = fastest(min(near, key=lambda v: abs(math.log2(v["K"] / key[2]))))[1]
                b_us = s_us = 0
        new.append((key, f"{{{key[0]}, {r['M']}, {r['K']}, {r['N']}, {p['kernel']}, "
                         f"{p['tile_cfg']}, {p['tile_n']}, {p['tile_m']}, {p['split_k']}, "
                         f"{b_us}, {s_us}}},"))
    for ln in kept:
        f = [int(v) for v in ln.strip("{},").split(",")[:4]]
        new.append((tuple(f), ln))
    order = {128: 0, 64: 1, 32: 2}
    new.sort(key=lambda t: (order[t[0][0]], t[0][1], t[0][2], t[0][3]))
    lines += [ln for _, ln in new]
    lines.append("// clang-format on")
    return "\n".join(lines) + "\n"


def _cold_note(r: dict) -> str:
    if r["weight_copies"] <= 1:
        return "warm: one copy of the weights"
    n = r["weight_copies"]
    return (f"cold: {n} rotating copies ({n * r['copy_mib']:.0f} MiB); each timed call's copy "
            f"was last read {n} calls ({(n - 1) * r['copy_mib']:.0f} MiB of other weights) earlier")


def _host_cpus() -> tuple[int, int, str]:
    """(threads to use, CPUs in this process's affinity mask, CPU model).  The
    thread count is the affinity mask, capped by OMP_NUM_THREADS where the
    host sets it (the GPU box's CPU share)."""
    n_aff = len(os.sched_getaffinity(0))
    n = n_aff
    try:
        cap = int(os.environ.get("OMP_NUM_THREADS", "0"))
        if cap > 0:
            n = min(n, cap)
    except ValueError:
        pass
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return max(1, n), n_aff, model


def cpu_baseline(case, budget_s: float = 12.0, max_calls: int = 40) -> dict:
    """The oracle's dequantise-then-matmul path on the host's cores: the N
    columns split into one contiguous chunk per thread (columns of a GEMM are
    independent), each chunk through oracle.reference_w4a16 with a
    single-threaded BLAS."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import w4a16_oracle as O
    from w4a16 import workloads as wl

    threads, n_aff, model = _host_cpus()
    X, W = wl.make_inputs(case)
    qw, s, z = O.quantize_weight(W.numpy(), case.G)
    Xn = X.numpy()
    bounds = np.linspace(0, case.N, threads + 1).astype(int)
    chunks = [(np.ascontiguousarray(qw[:, a:b]), np.ascontiguousarray(s[:, a:b]),
               np.ascontiguousarray(z[:, a:b])) for a, b in zip(bounds[:-1], bounds[1:]) if b > a]

    def run(pool):
        parts = list(pool.map(lambda c: O.reference_w4a16(Xn, c[0], c[1], c[2], case.G), chunks))
        return np.concatenate(parts, axis=1)

    times = []
    with threadpool_limits(limits=1), ThreadPoolExecutor(max_workers=len(chunks)) as pool:
        y = run(pool)                                  # warm-up
        ref = O.reference_w4a16(Xn, qw, s, z, case.G)
        assert np.array_equal(y.view(np.uint16), ref.view(np.uint16)) or \
            O.within_tolerance(y, ref).all()
        t_end = time.perf_counter() + budget_s
        while len(times) < max_calls and time.perf_counter() < t_end:
            t0 = time.perf_counter()
            run(pool)
            times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": case.bytes() / med / 1e9, "unit": "GB/s", "cores": len(chunks),
            "kind": "port",
            "sample": f"{len(times)} calls of oracle reference_w4a16 on the {case.name} inputs "
                      f"(numpy; N split over {len(chunks)} threads, BLAS 1 thread each), "
                      f"median {med * 1e3:.2f} ms/call",
            "ms_per_call": med * 1e3, "cpu_model": model, "host_cpus": n_aff}


# --------------------------------------------------------------------------- #
# the reference's benchmark (bench_gemm.py), reproduced                         #
# --------------------------------------------------------------------------- #
# bench_gemm.py:31-40
REF_DEFAULT_SHAPES = [(1, 4096, 4096), (1, 4096, 11008), (1, 11008, 4096), (64, 4096, 4096),
                      (256, 4096, 4096), (256, 4096, 11008), (256, 11008, 4096)]


def _ref_time_ms(fn, warmup: int = 25, iters: int = 100) -> float:
    """bench_gemm.py:43-58: median of `iters` calls, each bracketed by events on
    the current stream and a synchronize."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    for _ in range(iters):
        start.record()
        fn()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end))
    times.sort()
    return times[len(times) // 2]


def reference_row(M: int, K: int, N: int, G: int = 128, source: str = "bench_gemm") -> dict:
    """bench_gemm.py:70-99 for one shape: X, W ~ N(0, 1) fp16 on the GPU, W
    quantised (HIP kernel); fp16_matmul (hipBLASLt), dequant_then_matmul (HIP
    dequant + hipBLASLt) and the fused w4a16_matmul, each timed the
    reference's way; the same result keys."""
    import torch
    from w4a16 import dequant_then_matmul, fp16_matmul, quantize_weight, w4a16_matmul

    g = torch.Generator(device="cuda").manual_seed(M * 131 + K * 7 + N)
    X = torch.randn(M, K, dtype=torch.float16, device="cuda", generator=g)
    W = torch.randn(K, N, dtype=torch.float16, device="cuda", generator=g)
    qw, s, z = quantize_weight(W, G)
    t_fp16 = _ref_time_ms(lambda: fp16_matmul(X, W))
    t_dq = _ref_time_ms(lambda: dequant_then_matmul(X, qw, s, z, G))
    t_w4 = _ref_time_ms(lambda: w4a16_matmul(X, qw, s, z, G))
    flops = 2.0 * M * N * K
    ng = K // G
    b_w4 = M * K * 2 + (K // 8) * N * 4 + 2 * ng * N * 2 + M * N * 2
    b_fp16 = M * K * 2 + K * N * 2 + M * N * 2
    del W
    return {"M": M, "K": K, "N": N, "group_size": G, "source": source,
            "fp16_ms": t_fp16, "dequant_matmul_ms": t_dq, "w4a16_ms": t_w4,
            "w4a16_tflops": flops / (t_w4 * 1e-3) / 1e12,
            "fp16_tflops": flops / (t_fp16 * 1e-3) / 1e12,
            "w4a16_gbps": b_w4 / (t_w4 * 1e-3) / 1e9,
            "fp16_gbps": b_fp16 / (t_fp16 * 1e-3) / 1e9,
            "speedup_vs_fp16": t_fp16 / t_w4,
            "speedup_vs_dequant": t_dq / t_w4}


def to_markdown_table(results: list[dict]) -> str:
    """The reference's table (bench_gemm.py:102-117)."""
    header = (
        "| M | K | N | w4a16 (ms) | fp16 (ms) | dequant+mm (ms) | "
        "w4a16 TFLOPS | w4a16 GB/s | speedup vs fp16 | speedup vs dequant |\n"
        "|---|---|---|-----------|-----------|-----------------|"
        "--------------|------------|-----------------|--------------------|\n")
    rows = [f"| {r['M']} | {r['K']} | {r['N']} | {r['w4a16_ms']:.3f} | {r['fp16_ms']:.3f} | "
            f"{r['dequant_matmul_ms']:.3f} | {r['w4a16_tflops']:.1f} | {r['w4a16_gbps']:.0f} | "
            f"{r['speedup_vs_fp16']:.2f}x | {r['speedup_vs_dequant']:.2f}x |" for r in results]
    return header + "\n".join(rows) + "\n"


def reference_table(json_path: str | None) -> dict:
    from w4a16 import workloads as wl

    shapes = [(M, K, N, 128, "bench_gemm DEFAULT_SHAPES") for (M, K, N) in REF_DEFAULT_SHAPES]
    seen = {(M, K, N) for (M, K, N, _, _) in shapes}
    for c in wl.cases("C2", "C3", "C4", "C5"):
        if c.G == 128 and (c.M, c.K, c.N) not in seen:
            seen.add((c.M, c.K, c.N))
            shapes.append((c.M, c.K, c.N, 128, c.config))
    rows = []
    for M, K, N, G, src in shapes:
        r = reference_row(M, K, N, G, src)
        rows.append(r)
        print(f"M={M:<5} K={K:<6} N={N:<6} | w4a16 {r['w4a16_ms']:.4f}ms "
              f"({r['w4a16_tflops']:.1f} TF, {r['w4a16_gbps']:.0f} GB/s) | "
              f"fp16 {r['fp16_ms']:.4f}ms | dq {r['dequant_matmul_ms']:.4f}ms | "
              f"vs fp16 {r['speedup_vs_fp16']:.2f}x, vs dequant {r['speedup_vs_dequant']:.2f}x",
              file=sys.stderr, flush=True)
    print("\n" + to_markdown_table(rows), file=sys.stderr, flush=True)
    if json_path:
        with open(json_path, "w") as f:
            json.dump(rows, f, indent=1)
    return {"metric": "reference bench_gemm.py schema (warm weights, eager, median of 100)",
            "device": _device_name(), "rows": rows}


def _device_name() -> str:
    import torch

    return torch.cuda.get_device_name(0)


# --------------------------------------------------------------------------- #
# HBM traffic from rocprofv3 counters                                           #
# --------------------------------------------------------------------------- #
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic.json")

# --traffic-probe's workloads, in order: (key, config, M, K, N, G, calls, cold);
# config "X": a shape outside the BASELINE configs (C3-style weights).  The
# M <= 2 rows cover every kernel the planner picks there: the direct GEMV with
# 8 / 16 waves (C2, K = 14336), the skinny kernel's 32-column blocks (N =
# 6144), and the MFMA-dot GEMV on 128-column blocks and, split, on 64-column
# blocks with its reduction pass (N = 28672, C5, M = 2 at K = 14336).
PROBE = [("C2", "C2", 1, 4096, 4096, 128, 8, True),
         ("C3_M1_K4096_N6144", "C3", 1, 4096, 6144, 128, 4, True),
         ("C3_M1_K14336_N4096", "C3", 1, 14336, 4096, 128, 4, True),
         ("C3_M1_K4096_N28672", "C3", 1, 4096, 28672, 128, 4, True),
         ("C5_M1_K8192_N28672_G128", "C5", 1, 8192, 28672, 128, 4, True),
         ("C5_M1_K28672_N8192_G128", "C5", 1, 28672, 8192, 128, 4, True),
         ("M2_K14336_N4096", "X", 2, 14336, 4096, 128, 4, True),
         ("C3_M8_K4096_N4096", "C3", 8, 4096, 4096, 128, 4, True),
         ("C3_M32_K4096_N4096", "C3", 32, 4096, 4096, 128, 4, True),
         ("C3_M16_K4096_N28672", "C3", 16, 4096, 28672, 128, 4, True),
         ("C3_M32_K4096_N28672", "C3", 32, 4096, 28672, 128, 4, True),
         ("C4_M4096", "C4", 4096, 4096, 14336, 128, 3, False)]


def traffic_probe() -> None:
    """Kernels for the counter runs (FETCH_SIZE / WRITE_SIZE / SQ_*): a 256 MiB
    device copy three times (calibration), then each PROBE workload's calls
    with the default plans, each group preceded by one short spin kernel that
    marks where it starts."""
    import torch
    from w4a16 import w4a16_matmul
    from w4a16 import workloads as wl

    a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)                                   # calibration: 256 MiB read + written
    torch.cuda.synchronize()
    del a, b
    print("copy 256 MiB x3", flush=True)
    for key, cfg, M, K, N, G, calls, cold in PROBE:
        case = (wl.Case("X", M, K, N, G, 2) if cfg == "X" else
                [c for c in wl.CONFIGS[cfg] if (c.M, c.K, c.N, c.G) == (M, K, N, G)][0])
        X, W, Xd, layers, y, _, _ = _prepare(case, cold)
        torch.cuda.synchronize()
        torch.cuda._sleep(1000)                      # group marker
        for i in range(calls):
            l = layers[i % len(layers)]
            w4a16_matmul(Xd, l[0], l[1], l[2], case.G, out=y)
        torch.cuda.synchronize()
        del layers
        print(f"{key} x{calls}", flush=True)


def _counter_groups(path: str):
    """{counter: {workload: {kernel: [value per dispatch]}}} from a rocprofv3
    counter CSV of --traffic-probe, plus the calibration copies' values."""
    import csv

    disp = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            d = int(r["Dispatch_Id"])
            e = disp.setdefault(d, {"name": r["Kernel_Name"], "c": {}})
            e["c"][r["Counter_Name"]] = e["c"].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    out, calib = {}, {}
    gi = -1
    for d in sorted(disp):
        name, cs = disp[d]["name"], disp[d]["c"]
        if "copy" in name.lower() and gi < 0:
            for k, v in cs.items():
                calib.setdefault(k, []).append(v)
            continue
        if "spin_kernel" in name:
            gi += 1
            continue
        # the zeros check runs once per zeros tensor (its answer is cached),
        # not per call: left out like the quantize / pack / dequant kernels
        if gi < 0 or gi >= len(PROBE) or "w4a16" not in name or any(
                t in name for t in ("quantize", "pack", "dequant", "zeros_check")):
            continue
        for k, v in cs.items():
            out.setdefault(k, {}).setdefault(PROBE[gi][0], {}).setdefault(name, []).append(v)
    return out, calib


def traffic_from(fetch_csv: str, write_csv: str) -> dict:
    """HBM bytes per launch of each PROBE workload's kernels from
    --traffic-probe's counters.  FETCH_SIZE / WRITE_SIZE are in KiB per
    dispatch; each is scaled by what it reads for the calibration copy (the
    probe's first three copy dispatches, 256 MiB read and 256 MiB written
    each).  A workload's figure is its main kernel's (most dispatched, then
    longest name); a split-K reduction pass is listed beside it."""
    out = {"calibration": {"copy_bytes": 256 << 20}, "kernels": {}}
    for key, path, counter in (("fetch", fetch_csv, "FETCH_SIZE"),
                               ("write", write_csv, "WRITE_SIZE")):
        groups, calib = _counter_groups(path)
        copies = calib.get(counter, [])[:3]
        if len(copies) < 3:
            raise SystemExit(f"{path}: calibration copies not found")
        raw = sum(copies) / len(copies)
        scale = (256 << 10) / raw
        out["calibration"][f"{key}_size_kib_raw"] = raw
        out["calibration"][f"{key}_scale"] = scale
        for wkey, kernels in groups.get(counter, {}).items():
            e = out["kernels"].setdefault(wkey, {"launches": {}})
            for name, vals in kernels.items():
                k = e["launches"].setdefault(name, {"dispatches": len(vals)})
                k[f"{key}_kib_raw"] = sum(vals) / len(vals)
                k[f"{key}_bytes"] = k[f"{key}_kib_raw"] * 1024 * scale
    for e in out["kernels"].values():
        for k in e["launches"].values():
            k["bytes_per_launch"] = int(round(k.get("fetch_bytes", 0) + k.get("write_bytes", 0)))
        main = max(e["launches"], key=lambda n: ("reduce" not in n, e["launches"][n]["dispatches"]))
        e["kernel"] = main
        e["bytes_per_launch"] = e["launches"][main]["bytes_per_launch"]
    with open(TRAFFIC_JSON, "w") as f:
        json.dump(out, f, indent=1)
    return out


def _kernel_short(mangled: str) -> str:
    """`name<args>` of a kernel in this library's anonymous namespace from its
    mangled name (template arguments that are integer or bool literals only) or
    from the profiler's demangled one; the profiler leaves names with _Float16
    (DF16_) parameters mangled."""
    import re

    m = re.match(r"_ZN5w4a1612_GLOBAL__N_1(\d+)", mangled)
    if not m:                                    # already demangled by the profiler
        short = mangled.replace("w4a16::", "").replace("(anonymous namespace)::", "")
        return short.split("(")[0].replace("void ", "")
    n = int(m.group(1))
    at = m.end()
    name, rest = mangled[at:at + n], mangled[at + n:]
    if rest.startswith("I"):
        args = re.findall(r"L([ib])(\d+)E", rest[:rest.find("EE") + 2])
        name += "<" + ", ".join(("true" if v == "1" else "false") if t == "b" else v
                                for t, v in args) + ">"
    return name


def pmc_summary(paths) -> str:
    """Markdown table: per PROBE workload and kernel, each counter's average per
    dispatch over the --traffic-probe calls, from rocprofv3 --pmc CSVs."""
    rows = {}
    counters = []
    for p in paths:
        groups, _ = _counter_groups(p)
        for c, wl_ in groups.items():
            if c not in counters:
                counters.append(c)
            for wkey, kernels in wl_.items():
                for name, vals in kernels.items():
                    rows.setdefault((wkey, name), {})[c] = sum(vals) / len(vals)
    order = {k[0]: i for i, k in enumerate(PROBE)}
    lines = ["| workload | kernel | " + " | ".join(counters) + " |",
             "|---|---|" + "---|" * len(counters)]
    ordered = sorted(rows.items(), key=lambda kv: (order.get(kv[0][0], 99), kv[0][1]))
    for (wkey, name), cs in ordered:
        short = _kernel_short(name)
        lines.append(f"| {wkey} | `{short}` | " +
                     " | ".join(f"{cs[c]:,.0f}" if c in cs else "" for c in counters) + " |")
    need = ("SQ_WAVES", "SQ_INSTS_VMEM_RD", "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "SQ_INSTS_SALU",
            "SQ_INSTS_SMEM", "SQ_INSTS_LDS", "SQ_WAIT_INST_ANY", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES",
            "SQ_VALU_MFMA_BUSY_CYCLES")
    if all(c in counters for c in need):
        # per wave; SQ_BUSY_CYCLES counts for each of the 32 shader engines, the
        # MFMA busy cycles for each of the 1024 SIMDs
        lines += ["", "| workload | kernel | waves | VMEM_RD / wave | MFMA / wave | other VALU / wave "
                  "| SALU / wave | SMEM / wave | LDS / wave | WAIT_INST_ANY / WAVE_CYCLES "
                  "| busy cycles per SE | MFMA busy / busy |", "|---|---|" + "---|" * 10]
        for (wkey, name), cs in ordered:
            w = cs["SQ_WAVES"]
            per = {c: cs[c] / w for c in need}
            busy = cs["SQ_BUSY_CYCLES"] / 32
            lines.append(
                f"| {wkey} | `{_kernel_short(name)}` | {w:,.0f} | {per['SQ_INSTS_VMEM_RD']:.1f} | "
                f"{per['SQ_INSTS_MFMA']:.1f} | {per['SQ_INSTS_VALU'] - per['SQ_INSTS_MFMA']:.1f} | "
                f"{per['SQ_INSTS_SALU']:.1f} | {per['SQ_INSTS_SMEM']:.2f} | {per['SQ_INSTS_LDS']:.1f} | "
                f"{100 * cs['SQ_WAIT_INST_ANY'] / cs['SQ_WAVE_CYCLES']:.0f} % | {busy:,.0f} | "
                f"{100 * cs['SQ_VALU_MFMA_BUSY_CYCLES'] / 1024 / busy:.0f} % |")
    return "\n".join(lines)


def _traffic_for(workload: str):
    """HBM bytes per launch measured for a workload's kernel (profiles/traffic.json),
    or None when no measurement is recorded."""
    try:
        with open(TRAFFIC_JSON) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    return t.get("kernels", {}).get(workload, {}).get("bytes_per_launch")


def main() -> int:
    args = _args()
    if args.traffic_from:
        print(json.dumps(traffic_from(*args.traffic_from), indent=1))
        return 0
    if args.pmc_summary:
        print(pmc_summary(args.pmc_summary))
        return 0
    if args.trace_summary:
        print(trace_summary(args.trace_summary, args.steps, args.trace_last))
        return 0
    if args.decode_table:
        src = decode_table(args.decode_table)
        with open(DECODE_TABLE, "w") as f:
            f.write(src)
        n = sum(1 for ln in src.splitlines() if ln.startswith("{"))
        print(f"wrote {DECODE_TABLE} ({n} entries)")
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(this build targets a single MI355X: columns would shard with no "
              "communication, rows with one all-reduce of fp32 partial Y)",
              file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        return 2
    if args.traffic_probe:
        traffic_probe()
        return 0
    if args.empty_kernels:
        print(json.dumps(empty_kernels(args.steps, args.warmup)), flush=True)
        return 0
    if args.decode_scan:
        ints = lambda v: [int(t) for t in v.split(",")] if v else None
        decode_scan(args.decode_scan, ks=ints(args.decode_ks), ns=ints(args.decode_ns),
                    G=args.audit_g)
        return 0
    if args.planner_audit:
        shapes = AUDIT_SHAPES
        if args.audit_shapes:
            want = [tuple(map(int, s.split("x"))) for s in args.audit_shapes.split(",")]
            shapes = [a for a in AUDIT_SHAPES if (a[1], a[2]) in want] + [
                (f"{k}x{n}", k, n) for k, n in want if (k, n) not in
                {(a[1], a[2]) for a in AUDIT_SHAPES}]
        ms = [int(m) for m in args.audit_ms.split(",")] if args.audit_ms else AUDIT_MS
        print(planner_audit(shapes, ms, G=args.audit_g), flush=True)
        return 0
    if args.reference_table:
        print(json.dumps(reference_table(args.reference_json)), flush=True)
        return 0
    from w4a16 import workloads as wl

    graph = args.graph
    timing = ("HIP graph of the K calls, one replay, HIP events" if graph else
              "K eager calls queued behind a spin kernel, HIP events on their stream")
    c2 = wl.CONFIGS["C2"][0]
    head = bench_case(c2, args.steps, args.warmup, graph=graph, cold=True)
    ms = head["us"] / 1e3
    line = {
        "metric": "W4A16 GEMM HBM GB/s (M=1) & TFLOP/s (M=4096), % of MI355X roofline",
        "value": round(head["GB/s"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (uint4 weights, fp32 accumulate)",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, quantised on the GPU)",
        "config": {"workload": "C2 decode GEMV M=1 K=4096 N=4096 G=128",
                   "global_batch": 1, "parallelism": "none (1 GPU)",
                   "kernel": head["kernel"], "split_k": head["split_k"],
                   "tile_cfg": head["tile_cfg"], "weights": _cold_note(head), "timing": timing,
                   "queued_before_start": head["queued_before_start"],
                   "device": _device_name()},
        "roofline": {"bound": "hbm", "achieved": round(head["GB/s"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["GB/s"] / HBM_PEAK_GBS, 4),
                     "traffic": _traffic_for("C2")},
    }
    if not args.no_secondary:
        c4 = [c for c in wl.CONFIGS["C4"] if c.M == 4096][0]
        # steady state: after the light decode phase the chip's clock takes
        # ~100 calls of this load to settle under its power limit (25-call
        # chunks measured on MI355X: 493, 444, 426, 418, 416, then 411-417
        # µs per call), so 150 untimed calls (~60 ms), then 100 timed calls
        sec_steps, sec_warm = max(100, args.steps // 2), max(150, args.warmup // 2)
        sec = bench_case(c4, sec_steps, sec_warm, graph=SECONDARY_GRAPH, cold=False)
        line["secondary"] = {
            "metric": "TFLOP/s, C4 prefill M=4096 K=4096 N=14336 G=128",
            "value": round(sec["TFLOP/s"], 2), "unit": "TFLOP/s", "us": round(sec["us"], 2),
            "kernel": sec["kernel"], "tile_cfg": sec["tile_cfg"], "tile": sec["tile"],
            "timing": f"{sec['steps']} calls in one HIP graph replay after {sec_warm} untimed "
                      "calls, HIP events",
            "roofline": {"bound": "mfma", "achieved": round(sec["TFLOP/s"], 2),
                         "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(sec["TFLOP/s"] / FP16_PEAK_TFLOPS, 4),
                         "traffic": _traffic_for("C4_M4096")},
            "dense_fp16": dense_fp16_case(c4, sec_steps, sec_warm),
        }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(c2)
    if args.sweep:
        rows = []
        for case in wl.cases("C2", "C3", "C4", "C5"):
            # prefill-sized calls (M >= 64) as one graph replay, like the
            # secondary line; decode-sized calls eager behind the spin
            r = bench_case(case, max(20, args.steps // 4), 5, graph=graph or case.M >= 64,
                           cold=case.M < 64)
            rows.append(r)
            print(f"{r['case']:<32} {r['kernel']:>6} cfg={r['tile_cfg']:<2} "
                  f"split={r['split_k']:<3} {r['us']:9.2f} us {r['GB/s']:8.1f} GB/s "
                  f"{r['TFLOP/s']:8.2f} TFLOP/s", file=sys.stderr, flush=True)
        seen = set()
        for case in wl.cases("C2", "C4", "C5"):
            if (case.K, case.N, case.G) in seen:
                continue
            seen.add((case.K, case.N, case.G))
            r = bench_quantize(case, max(20, args.steps // 4), 3)
            rows.append(r)
            print(f"{r['case']:<32} {r['us']:9.2f} us {r['GB/s']:8.1f} GB/s (W read + packed "
                  "written)", file=sys.stderr, flush=True)
        if args.sweep_json:
            with open(args.sweep_json, "w") as f:
                json.dump(rows, f, indent=1)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
