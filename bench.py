"""Benchmark of the gfx950 K-quant matvec path (one MI355X).

Headline: Q4_K matvec, N=17408 rows x K=5120 columns,
batch 1, achieved HBM GB/s on packed-weight bytes (17408*20*144 =
50,135,040 B per call) and us/call.  A "step" is one matvec call.

Timing: weights for NCOPIES distinct matrices (> the 256 MB Infinity Cache)
stay resident in HBM; W warmup calls, then K calls back to back on the
library's compute stream, bracketed by HIP events recorded on that same
stream, each call reading the next copy.  The CPU baseline times the
oracle's restatement of the reference CPU path (quant.rs dequantisation
followed by the sequential f32 host dot) on the host cores.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--sweep] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "memory-aware-inference_amd"))

import si_hip  # noqa: E402

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the headline kernel from the two rocprofv3 --pmc
# passes (FETCH_SIZE, WRITE_SIZE) scaled by a copy of known size
TRAFFIC_PROFILE = REPO / "profiles" / "q4k_matvec_mfma_17408x5120_traffic.md"
METRIC = "Q4_K matvec achieved HBM GB/s (% of peak) + µs/call at 17408×5120, batch 1"
NCOPIES = 8


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def time_matvec(ctx, ggml_type: int, rows: int, cols: int, steps: int, warmup: int,
                copies: int = NCOPIES, seed: int = 17) -> dict:
    nbytes = rows * (cols // 256) * si_hip.BLOCK_BYTES[ggml_type]
    weights = []
    for c in range(copies):
        w = si_hip.synth_matrix(ggml_type, seed=seed + c, rows=rows, cols=cols, threads=16)
        weights.append(ctx.upload_quant_weight_private(w, ggml_type))
        del w
    x = si_hip.synth_normal(seed, cols)
    d_x = ctx.device_alloc(cols * 4)
    d_y = ctx.device_alloc(rows * 4)
    ctx.to_device(d_x, x)
    lib = si_hip.lib()
    import ctypes as C
    harr = (C.c_void_p * copies)(*[w.handle.value for w in weights])
    rc = lib.si_hip_quant_matvec_device_repeat(ctx.handle, harr, copies, rows, cols,
                                               C.c_void_p(d_x), C.c_void_p(d_y), warmup)
    if rc:
        raise si_hip.HipError(rc, si_hip.last_error())
    ctx.synchronize()
    ctx.event_record(0)
    rc = lib.si_hip_quant_matvec_device_repeat(ctx.handle, harr, copies, rows, cols,
                                               C.c_void_p(d_x), C.c_void_p(d_y), steps)
    if rc:
        raise si_hip.HipError(rc, si_hip.last_error())
    ctx.event_record(1)
    ms = ctx.event_elapsed_ms(0, 1)
    ctx.synchronize()
    ctx.device_free(d_x)
    ctx.device_free(d_y)
    for w in weights:
        w.free()
    us = ms * 1000.0 / steps
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"rows": rows, "cols": cols, "ggml_type": ggml_type, "bytes_per_call": nbytes,
            "us_per_call": round(us, 3), "gb_per_s": round(gbs, 1),
            "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4)}


def profiled_traffic() -> int | None:
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_baseline(rows: int, cols: int, budget_s: float = 10.0) -> dict:
    """Reference CPU path (oracle restatement of quant.rs + host dot), 1 thread."""
    sys.path.insert(0, str(REPO / "tests"))
    import oracle_lib  # the checker library; only this leg of the benchmark uses it
    w = si_hip.synth_matrix(12, seed=99, rows=rows, cols=cols, threads=16)
    x = si_hip.synth_normal(99, cols)
    lib = oracle_lib.lib()
    import ctypes as C
    y = np.empty(rows, np.float32)
    bp = w.ctypes.data_as(C.POINTER(C.c_uint8))
    xp = x.ctypes.data_as(C.POINTER(C.c_float))
    yp = y.ctypes.data_as(C.POINTER(C.c_float))
    calls = 0
    t0 = time.perf_counter()
    while True:
        rc = lib.kq_matvec_ref(12, bp, w.size, rows, cols, xp, yp, None, None, 1)
        assert rc == 0
        calls += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = (time.perf_counter() - t0) / calls
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(w.size / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "us_per_call": round(dt * 1e6, 1),
            "sample": f"{calls} full Q4_K {rows}x{cols} calls (quant.rs dequant + sequential f32 "
                      f"dot), oracle/kquant_ref.c -O2 -ffp-contract=off, {model}"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sweep", action="store_true", help="also time the batch-1 shape sweep")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-probe", action="store_true",
                    help="also time device-to-device copies of the matrix size (the yardstick "
                         "that scales HBM traffic counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(see DESIGN.md for how the matvec would shard)", file=sys.stderr)
        return 2

    ctx = si_hip.HipContext(0)
    rows, cols = 17408, 5120
    log(f"timing Q4_K {rows}x{cols}, {args.steps} steps, {NCOPIES} resident copies")
    head = time_matvec(ctx, 12, rows, cols, args.steps, args.warmup)
    log(f"  {head['us_per_call']} us/call, {head['gb_per_s']} GB/s")
    out = {
        "metric": METRIC,
        "value": head["gb_per_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_call"] / 1000.0, 6),
        "us_per_call": head["us_per_call"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights (u8 packed) x f32 activations, f32 accumulate",
        "data": "synthetic (seeded generator, BASELINE.json config 2)",
        "config": {"workload": "Q4_K matvec N=17408 x K=5120, batch 1", "rows": rows,
                   "cols": cols, "batch": 1, "weight_copies": NCOPIES,
                   "bytes_per_call": head["bytes_per_call"]},
        "roofline": {"bound": "hbm", "achieved": head["gb_per_s"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": head["frac_of_peak"],
                     "traffic": profiled_traffic()},
    }
    if args.copy_probe:
        nbytes = head["bytes_per_call"]
        src, dst = ctx.device_alloc(nbytes), ctx.device_alloc(nbytes)
        for _ in range(args.warmup):
            ctx.device_copy(dst, src, nbytes)
        ctx.synchronize()
        ctx.event_record(0)
        for _ in range(args.steps):
            ctx.device_copy(dst, src, nbytes)
        ctx.event_record(1)
        ms = ctx.event_elapsed_ms(0, 1)
        ctx.synchronize()
        ctx.device_free(src)
        ctx.device_free(dst)
        us = ms * 1000.0 / args.steps
        out["copy_probe"] = {"bytes_read_per_copy": nbytes, "us_per_copy": round(us, 3),
                             "gb_per_s_read": round(nbytes / (us * 1e-6) / 1e9, 1)}
        log(f"  copy probe {nbytes} B: {us:.3f} us")
    if args.sweep:
        sweep = []
        for r, c in ((5120, 5120), (17408, 5120), (5120, 17408), (1024, 5120)):
            res = time_matvec(ctx, 12, r, c, args.steps, args.warmup)
            log(f"  sweep {r}x{c}: {res['us_per_call']} us, {res['gb_per_s']} GB/s")
            sweep.append(res)
        out["sweep"] = sweep
    ctx.close()
    if not args.no_cpu:
        log("timing the CPU baseline")
        out["cpu_baseline"] = cpu_baseline(rows, cols, args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
