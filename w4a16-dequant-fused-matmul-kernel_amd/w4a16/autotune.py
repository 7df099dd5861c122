"""Measured plan selection per GEMM shape (opt-in).

The reference picks its Triton kernel's tiling at run time: ``@triton.autotune``
over a list of configs keyed on ``(M, N, K, group_size)`` times every config on
the first call of a shape and keeps the fastest (w4a16-kernel/src/w4a16/
triton_kernel.py:41-62).  Here the library's static planner (``capi.cpp``
``make_plan``, thresholds measured on MI355X) chooses by default, so a call
never pays a tuning pass and the kernel choice does not depend on timing
noise.  With autotuning on, the first call of each shape (device, M, N, K, G,
row strides, zero-point form) instead times the planner's choice and its
neighbours -- other kernel families, column-block widths, wave counts, tile
heights and k-splits -- on the caller's own tensors and keeps the fastest
plan for every later call of that shape.

* ``enable(True / False)``, or the environment variable ``W4A16_AUTOTUNE=1``;
* ``W4A16_AUTOTUNE_CACHE=/path/file.json``: tuned plans are loaded from and
  saved to that file (keyed by device name as well), so a serving process
  tunes once per machine;
* calls made under HIP-graph capture are never tuned (a tuning pass launches
  and synchronises); they use a plan already tuned, else the static planner's;
* every candidate is a plan the library validates like any explicit plan; all
  of them meet the same parity tests, but two plans may differ in the last
  bits where they sum k in a different order (split-K, wave counts), so a
  tuned process is deterministic per shape but need not match the static
  planner's bits.
"""
from __future__ import annotations

import json
import os
import statistics
import threading

import torch

from . import _lib
from . import _runtime as rt

__all__ = ["enable", "enabled", "clear", "tuned", "candidates", "time_plans"]

_LOCK = threading.Lock()
_STATE = {"on": os.environ.get("W4A16_AUTOTUNE", "") not in ("", "0"), "loaded": False}
_CACHE: dict[str, dict] = {}


def enable(flag: bool = True) -> None:
    """Turn measured plan selection on or off for this process."""
    _STATE["on"] = bool(flag)


def enabled() -> bool:
    return _STATE["on"]


def clear() -> None:
    """Forget every tuned plan (the cache file is left as it is)."""
    with _LOCK:
        _CACHE.clear()


def tuned() -> dict[str, dict]:
    """The tuned plans so far: key -> {"plan": fields, "us": time, "static_us": ...}."""
    with _LOCK:
        return {k: dict(v) for k, v in _CACHE.items()}


def _plan_fields(p: _lib.Plan) -> dict:
    return {name: int(getattr(p, name)) for name, _ in p._fields_}


def _plan_from(fields: dict) -> _lib.Plan:
    p = _lib.Plan()
    for name, _ in p._fields_:
        setattr(p, name, int(fields.get(name, 0)))
    return p


def candidates(M: int, N: int, K: int, G: int) -> list[tuple[str, _lib.Plan]]:
    """The static plan first, then every other plan the library has for the
    shape: GEMV column widths, wave counts, staging and MFMA-dot forms and
    k-splits (M <= 8); skinny block widths and row groups (M <= 64); streamed
    prefill tiles (32 / 64 / 128 rows, one or two k-slices) and their k-splits,
    and the register-staged tilings where K % 256 != 0.  Plans a shape cannot
    take are left for the library to refuse (W4A16_ERR_BAD_PLAN)."""
    out: list[tuple[str, _lib.Plan]] = []
    seen = set()

    def add(label: str, p: _lib.Plan) -> None:
        key = (p.kernel, p.split_k, p.tile_cfg, p.tile_m, p.tile_n)
        if key not in seen:
            seen.add(key)
            out.append((label, p))

    def plan(kernel: int, split: int = 0):
        try:
            return _lib.plan(M, N, K, G, kernel, split)
        except RuntimeError:
            return None

    add("static", _lib.plan(M, N, K, G))
    if M == 0 or N == 0 or K == 0:
        return out
    if M <= 8 and N % 4 == 0 and G % 32 == 0:
        # column blocks that leave at least an eighth of the CUs a block;
        # k-splits 2 and 4 (8 from K = 16384)
        widths = [c for c in (16, 32, 64, 128, 256) if c == 16 or (N + c - 1) // c >= 32]
        splits = (1, 2, 4, 8) if K >= 16384 else (1, 2, 4)
        for cfg in ((1, 2, 4, 5, 6, 7) if M <= 2 else (1,)):
            for cols in ([c for c in widths if c in (64, 128)] if cfg >= 6 else widths):
                for split in splits:
                    if split > K // 8:
                        continue
                    p = plan(_lib.KERNEL_GEMV, split)
                    if p is None:
                        continue
                    p.tile_n, p.tile_cfg = cols, cfg
                    add(f"gemv cfg={cfg} cols={cols} split={p.split_k}", p)
    if M <= 64 and G % 32 == 0:
        whole = (M + 15) // 16 * 16
        for rows in sorted({whole, 16, 8}):
            for cfg, cols in ((0, 16), (2, 32), (3, 64)):
                if (cfg == 2 and (rows > 32 or N % 2)) or (cfg == 3 and (rows > 16 or N % 4)):
                    continue
                if rows == 8 and not 9 <= M <= 16:
                    continue
                p = plan(_lib.KERNEL_SKINNY)
                if p is None:
                    continue
                p.tile_cfg, p.tile_m, p.tile_n = cfg, rows, cols
                add(f"skinny cfg={cfg} rows={rows}", p)
    if N % 4 == 0 and G % 32 == 0:
        if K % 256 == 0:
            cfgs = (12, 13) if M <= 64 else ((13, 11, 14) if M <= 512 else (11, 14))
        else:
            cfgs = (7, 6, 1, 2) if K % 128 == 0 else ((7, 1, 2) if K % 64 == 0 else (1, 2))
        for cfg in cfgs:
            splits = (1, 2, 3, 4, 6, 8) if cfg in _lib.MFMA_SPLIT_CONFIGS else (1,)
            for split in splits:
                if split > 1 and K // 64 < 4 * split:
                    continue
                p = plan(_lib.KERNEL_MFMA, split)
                if p is None:
                    continue
                p.tile_cfg = cfg
                p.tile_m, p.tile_n = {1: (128, 256), 2: (32, 512), 6: (128, 256), 7: (128, 256),
                                      11: (128, 256), 12: (32, 256), 13: (64, 256),
                                      14: (128, 256)}[cfg]
                add(f"mfma cfg={cfg} split={p.split_k}", p)
    return out


def time_plans(x, qweight, scales, zeros, G: int, plans, reps: int = 3,
               budget_us: float = 400.0, ldy: int | None = None) -> list[float]:
    """Median µs per call of each plan on these tensors (warm weights; calls on
    the current stream, HIP events; repetitions interleaved across the plans).
    The output is a scratch tensor with row stride `ldy` (default N), so a plan
    is tried on the caller's layout.  A plan the library refuses gets +inf.
    Each repetition is a run of calls of about `budget_us`."""
    from .hip_kernel import w4a16_matmul_planned

    M, K = x.shape
    N = qweight.shape[1]
    ldy = N if ldy is None else ldy
    y = torch.empty((M, ldy), dtype=torch.float16, device=x.device)[:, :N]
    stream = torch.cuda.current_stream(x.device)
    live, est = [], []
    for p in plans:
        try:
            for _ in range(2):
                w4a16_matmul_planned(x, qweight, scales, zeros, G, p, out=y)
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record(stream)
            w4a16_matmul_planned(x, qweight, scales, zeros, G, p, out=y)
            t1.record(stream)
            t1.synchronize()
            live.append(True)
            est.append(max(t0.elapsed_time(t1) * 1e3, 1.0))
        except RuntimeError:
            live.append(False)
            est.append(float("inf"))
    times: list[list[float]] = [[] for _ in plans]
    for _ in range(reps):
        for i, p in enumerate(plans):
            if not live[i]:
                continue
            n = max(3, min(200, int(budget_us / est[i])))
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record(stream)
            for _ in range(n):
                w4a16_matmul_planned(x, qweight, scales, zeros, G, p, out=y)
            t1.record(stream)
            t1.synchronize()
            times[i].append(t0.elapsed_time(t1) * 1e3 / n)
    return [statistics.median(t) if t else float("inf") for t in times]


def _cache_path() -> str | None:
    return os.environ.get("W4A16_AUTOTUNE_CACHE") or None


def _load_file() -> None:
    if _STATE["loaded"]:
        return
    _STATE["loaded"] = True
    path = _cache_path()
    if not path or not os.path.exists(path):
        return
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return
    if isinstance(data, dict):
        _CACHE.update({k: v for k, v in data.items() if isinstance(v, dict) and "plan" in v})


def _save_file() -> None:
    path = _cache_path()
    if not path:
        return
    tmp = path + ".tmp"
    with open(tmp, "w") as f:
        json.dump(_CACHE, f, indent=1, sort_keys=True)
    os.replace(tmp, path)


def _key(x, M, N, K, G, ldx, ldy, any_zeros) -> str:
    dev = x.device.index if x.device.index is not None else torch.cuda.current_device()
    return (f"{torch.cuda.get_device_name(dev)}|{M}x{N}x{K}|G{G}|ld{ldx},{ldy}"
            f"|{'anyz' if any_zeros else 'intz'}")


def plan_for_call(x, qweight, scales, zeros, G: int, M: int, N: int, K: int, ldx: int, ldy: int,
                  any_zeros: bool):
    """The tuned plan of this call's shape (tuning it now if it is new), or None
    under graph capture when the shape has not been tuned."""
    key = _key(x, M, N, K, G, ldx, ldy, any_zeros)
    with _LOCK:
        _load_file()
        hit = _CACHE.get(key)
    if hit is not None:
        return _plan_from(hit["plan"])
    if torch.cuda.is_current_stream_capturing():
        return None
    cands = candidates(M, N, K, G)
    plans = [p for _, p in cands]
    us = time_plans(x, qweight, scales, zeros, G, plans, ldy=ldy)
    best = min(range(len(plans)), key=lambda i: us[i])
    entry = {"plan": _plan_fields(plans[best]), "label": cands[best][0], "us": us[best],
             "static_us": us[0], "candidates": len(plans)}
    with _LOCK:
        _CACHE[key] = entry
        _save_file()
    return _plan_from(entry["plan"])
