"""Benchmark of the W4A16 fused dequant-GEMM on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--sweep]

Prints ONE JSON line.  Headline (``value``): HBM GB/s of the decode GEMV at
BASELINE config C2 (M=1, K=N=4096, G=128) -- algorithmic bytes per call
(2MK + 4(K/8)N + 4(K/G)N + 2MN, reference bench_gemm.py:61-67) over the average
kernel time.  Timing:

* weights cold: the call cycles over enough copies of (qweight, scales, zeros)
  that they total > 512 MiB, so the 256 MiB Infinity Cache cannot hold them;
* the K timed calls are captured once into a HIP graph and replayed, bracketed
  by HIP events recorded on the stream the kernels run on, so host launch
  overhead is not in the figure; ``ms_per_step`` = event time / K;
* ``secondary``: TFLOP/s of the prefill MFMA GEMM at C4 M=4096 (2MNK flops);
* ``cpu_baseline``: the CPU oracle's dequantise-then-matmul path
  (``oracle/w4a16_oracle.reference_w4a16``, a numpy port of the reference's
  reference.py:18-40) on the same C2 inputs, single-threaded, timed on this
  host over a bounded number of calls.
"""
from __future__ import annotations

import argparse
import json
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
    ap.add_argument("--eager", action="store_true", help="time eager launches, not a graph")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run the workload for rocprofv3 --pmc: a 256 MiB copy (calibration), "
                         "8 cold C2 decode calls, 3 C4 M=4096 prefill calls; no timing")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write profiles/traffic.json from the counter_collection.csv files "
                         "of two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of "
                         "--traffic-probe")
    return ap.parse_args()


def _time_calls(fns, steps: int, warmup: int, graph: bool):
    """Average ms per call of `fns` (cycled), HIP events on the launch stream."""
    import torch

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(max(warmup, len(fns))):
            fns[i % len(fns)]()
    stream.synchronize()
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(steps):
                fns[i % len(fns)]()
        with torch.cuda.stream(stream):
            g.replay()                      # one untimed replay
        stream.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        start.record(stream)
        if graph:
            g.replay()
        else:
            for i in range(steps):
                fns[i % len(fns)]()
        end.record(stream)
    end.synchronize()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


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
    layers = [(qw, s, z)] + [(qw.clone(), s.clone(), z.clone()) for _ in range(ncopy - 1)]
    y = torch.empty(case.M, case.N, dtype=torch.float16, device="cuda")
    return X, W, Xd, layers, y, ncopy


def bench_case(case, steps: int, warmup: int, graph: bool = True, cold: bool = True) -> dict:
    from w4a16 import w4a16_matmul
    from w4a16.hip_kernel import plan_for

    X, W, Xd, layers, y, ncopy = _prepare(case, cold)
    fns = [(lambda l=l: w4a16_matmul(Xd, l[0], l[1], l[2], case.G, out=y)) for l in layers]
    ms = _time_calls(fns, steps, warmup, graph)
    p = plan_for(case.M, case.N, case.K, case.G).as_dict()
    us = ms * 1e3
    gbs = case.bytes() / (ms * 1e-3) / 1e9
    tflops = case.flops() / (ms * 1e-3) / 1e12
    return {"case": case.name, "M": case.M, "K": case.K, "N": case.N, "G": case.G,
            "us": us, "GB/s": gbs, "TFLOP/s": tflops, "weight_copies": ncopy,
            "kernel": p["kernel_name"], "split_k": p["split_k"], "tile": [p["tile_m"], p["tile_n"]],
            "grid": [p["grid_x"], p["grid_y"]], "bytes": case.bytes(), "flops": case.flops()}


def cpu_baseline(case, budget_s: float = 12.0, max_calls: int = 40) -> dict:
    """The oracle's dequantise-then-matmul path on the host, one thread."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import w4a16_oracle as O
    from w4a16 import workloads as wl

    X, W = wl.make_inputs(case)
    qw, s, z = O.quantize_weight(W.numpy(), case.G)
    Xn = X.numpy()
    times = []
    with threadpool_limits(limits=1):
        O.reference_w4a16(Xn, qw, s, z, case.G)       # warm-up
        t_end = time.perf_counter() + budget_s
        while len(times) < max_calls and time.perf_counter() < t_end:
            t0 = time.perf_counter()
            O.reference_w4a16(Xn, qw, s, z, case.G)
            times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": case.bytes() / med / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{len(times)} calls of oracle reference_w4a16 on the {case.name} inputs "
                      f"(numpy, 1 thread), median {med * 1e3:.2f} ms/call",
            "ms_per_call": med * 1e3}


TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic.json")


def traffic_probe() -> None:
    """Kernels for the HBM-traffic counters (FETCH_SIZE / WRITE_SIZE)."""
    import torch
    from w4a16 import w4a16_matmul
    from w4a16 import workloads as wl

    a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)                                   # calibration: 256 MiB read + written
    torch.cuda.synchronize()
    print("copy 256 MiB x3", flush=True)
    c2 = wl.CONFIGS["C2"][0]
    X, W, Xd, layers, y, _ = _prepare(c2, True)
    for i in range(8):
        l = layers[i % len(layers)]
        w4a16_matmul(Xd, l[0], l[1], l[2], c2.G, out=y)
    torch.cuda.synchronize()
    print("C2 x8", flush=True)
    del layers
    c4 = [c for c in wl.CONFIGS["C4"] if c.M == 4096][0]
    X, W, Xd, layers, y, _ = _prepare(c4, False)
    for _ in range(3):
        w4a16_matmul(Xd, layers[0][0], layers[0][1], layers[0][2], c4.G, out=y)
    torch.cuda.synchronize()
    print("C4 M=4096 x3", flush=True)


def _counter_rows(path: str, counter: str):
    """(dispatch id, kernel name, value) per dispatch from a rocprofv3 counter CSV."""
    import csv

    rows = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            d = int(r["Dispatch_Id"])
            name, v = r["Kernel_Name"], float(r["Counter_Value"])
            rows[d] = (name, rows.get(d, (name, 0.0))[1] + v)
    return [(d, n, v) for d, (n, v) in sorted(rows.items())]


def traffic_from(fetch_csv: str, write_csv: str) -> dict:
    """HBM bytes per launch of the C2 and C4 GEMM kernels from --traffic-probe's
    counters.  FETCH_SIZE / WRITE_SIZE are in KiB per dispatch; each is scaled by
    what it reads for the calibration copy (the probe's first three copy
    dispatches, 256 MiB read and 256 MiB written each)."""
    out = {"calibration": {"copy_bytes": 256 << 20}, "kernels": {}}
    per = {}
    for key, path, counter in (("fetch", fetch_csv, "FETCH_SIZE"),
                               ("write", write_csv, "WRITE_SIZE")):
        rows = _counter_rows(path, counter)
        copies = [v for _, n, v in rows if "copy" in n.lower()][:3]
        if len(copies) < 3:
            raise SystemExit(f"{path}: calibration copies not found")
        raw = sum(copies) / len(copies)
        scale = (256 << 10) / raw
        out["calibration"][f"{key}_size_kib_raw"] = raw
        out["calibration"][f"{key}_scale"] = scale
        gemm = [(n, v) for _, n, v in rows if "w4a16" in n
                and not any(t in n for t in ("quantize", "pack", "dequant"))]
        if len(gemm) != 11:
            raise SystemExit(f"{path}: expected 8 C2 + 3 C4 GEMM dispatches, got {len(gemm)}")
        per[key] = {"C2": (gemm[0][0], gemm[:8]), "C4_M4096": (gemm[8][0], gemm[8:])}
        for wkey, (name, ds) in per[key].items():
            e = out["kernels"].setdefault(wkey, {"kernel": name})
            e[f"{key}_kib_raw"] = sum(v for _, v in ds) / len(ds)
            e[f"{key}_bytes"] = e[f"{key}_kib_raw"] * 1024 * scale
    for e in out["kernels"].values():
        e["bytes_per_launch"] = int(round(e["fetch_bytes"] + e["write_bytes"]))
    with open(TRAFFIC_JSON, "w") as f:
        json.dump(out, f, indent=1)
    return out


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
    if args.traffic_probe:
        traffic_probe()
        return 0
    if args.traffic_from:
        print(json.dumps(traffic_from(*args.traffic_from), indent=1))
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
    from w4a16 import workloads as wl

    graph = not args.eager
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
                   "weights": f"cold: {head['weight_copies']} rotating copies",
                   "timing": "HIP graph of K calls, HIP events" if graph else "eager, HIP events"},
        "roofline": {"bound": "hbm", "achieved": round(head["GB/s"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["GB/s"] / HBM_PEAK_GBS, 4),
                     "traffic": _traffic_for("C2")},
    }
    if not args.no_secondary:
        c4 = [c for c in wl.CONFIGS["C4"] if c.M == 4096][0]
        # steady state: 10 untimed calls (the clock settles under the MFMA
        # load after the light decode phase), then 50 timed calls (~25 ms)
        sec = bench_case(c4, max(50, args.steps // 4), max(10, args.warmup // 2), graph=graph,
                         cold=False)
        line["secondary"] = {
            "metric": "TFLOP/s, C4 prefill M=4096 K=4096 N=14336 G=128",
            "value": round(sec["TFLOP/s"], 2), "unit": "TFLOP/s", "us": round(sec["us"], 2),
            "kernel": sec["kernel"], "tile": sec["tile"],
            "roofline": {"bound": "mfma", "achieved": round(sec["TFLOP/s"], 2),
                         "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(sec["TFLOP/s"] / FP16_PEAK_TFLOPS, 4),
                         "traffic": _traffic_for("C4_M4096")},
        }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(c2)
    if args.sweep:
        rows = []
        for case in wl.cases("C2", "C3", "C4", "C5"):
            r = bench_case(case, max(20, args.steps // 4), 5, graph=graph,
                           cold=case.M < 64)
            rows.append(r)
            print(f"{r['case']:<32} {r['kernel']:>5} split={r['split_k']:<3} "
                  f"{r['us']:9.2f} us {r['GB/s']:8.1f} GB/s {r['TFLOP/s']:8.2f} TFLOP/s",
                  file=sys.stderr, flush=True)
        if args.sweep_json:
            with open(args.sweep_json, "w") as f:
                json.dump(rows, f, indent=1)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
