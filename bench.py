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

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
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
# every timed leg cycles through distinct resident weight copies whose bytes
# together exceed the 256 MB Infinity Cache (MALL) with room to spare, so
# that its rate is an HBM rate, not a cache rate
RESIDENT_MIN_BYTES = 300_000_000
WARM_MS = 20.0  # least warm-up of every timed leg (an idle GPU clocks down)


def copies_for(bytes_per_call: int, least: int = 2) -> int:
    """Distinct copies a leg rotates: more than RESIDENT_MIN_BYTES in all."""
    return max(least, RESIDENT_MIN_BYTES // bytes_per_call + 1)


def residency(bytes_per_call: int, copies: int) -> dict:
    return {"weight_copies": copies, "resident_bytes": bytes_per_call * copies}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def time_matvec(ctx, ggml_type: int, rows: int, cols: int, steps: int, warmup: int,
                copies: int | None = None, seed: int = 17, detail: bool = False,
                graph: bool = True) -> dict:
    nbytes = rows * (cols // 256) * si_hip.BLOCK_BYTES[ggml_type]
    if copies is None:
        copies = copies_for(nbytes)
    weights = []
    host0 = None  # copy 0's host bytes, for the borrowed-bytes timing
    for c in range(copies):
        w = si_hip.synth_matrix(ggml_type, seed=seed + c, rows=rows, cols=cols, threads=16)
        weights.append(ctx.upload_quant_weight_private(w, ggml_type))
        if c == 0 and detail:
            host0 = w
        del w
    x = si_hip.synth_normal(seed, cols)
    d_x = ctx.device_alloc(cols * 4)
    d_y = ctx.device_alloc(rows * 4)
    ctx.to_device(d_x, x)
    lib = si_hip.lib()
    import ctypes as C
    harr = (C.c_void_p * copies)(*[w.handle.value for w in weights])
    # at least `warmup` calls and WARM_MS of them
    t0 = time.perf_counter()
    warm_calls = 0
    while warm_calls < warmup or (time.perf_counter() - t0) * 1e3 < WARM_MS:
        n = max(warmup - warm_calls, 25)
        rc = lib.si_hip_quant_matvec_device_repeat(ctx.handle, harr, copies, rows, cols,
                                                   C.c_void_p(d_x), C.c_void_p(d_y), n)
        if rc:
            raise si_hip.HipError(rc, si_hip.last_error())
        ctx.synchronize()
        warm_calls += n
    warm_ms = (time.perf_counter() - t0) * 1e3
    ctx.event_record(0)
    rc = lib.si_hip_quant_matvec_device_repeat(ctx.handle, harr, copies, rows, cols,
                                               C.c_void_p(d_x), C.c_void_p(d_y), steps)
    if rc:
        raise si_hip.HipError(rc, si_hip.last_error())
    ctx.event_record(1)
    ms = ctx.event_elapsed_ms(0, 1)
    ctx.synchronize()
    extra = {}
    if graph:
        graph_ms = time_graph_repeat(ctx, lib, harr, copies, rows, cols, d_x, d_y, steps, warmup)
        extra = {"graph_us_per_call": round(graph_ms * 1000.0, 3),
                 "graph_gb_per_s": round(nbytes / (graph_ms * 1e-3) / 1e9, 1)}
    if detail:
        extra.update(call_detail(ctx, lib, harr, weights, rows, cols, x, d_x, d_y, steps, host0))
        if GRAPHS:  # (the probe's launches are replayed from a graph)
            extra["floor"] = stream_floor(ctx, lib, harr, copies, rows, cols, nbytes, steps,
                                          warmup, ggml_type)
    ctx.device_free(d_x)
    ctx.device_free(d_y)
    for w in weights:
        w.free()
    us = ms * 1000.0 / steps
    gbs = nbytes / (us * 1e-6) / 1e9
    out = {"rows": rows, "cols": cols, "ggml_type": ggml_type, "bytes_per_call": nbytes,
           "us_per_call": round(us, 3), "gb_per_s": round(gbs, 1),
           "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4), **residency(nbytes, copies),
           "warmup_calls": warm_calls, "warmup_ms": round(warm_ms, 1)}
    out.update(extra)
    return out


def stream_floor(ctx, lib, harr, copies, rows, cols, nbytes, steps: int, warmup: int,
                 ggml_type: int = 12) -> dict:
    """Back-to-back launches of si_hip_stream_probe over the same resident
    copies: the matvec kernel's weight copies alone (its grid, 12 waves per
    CU, 16-row x 64-byte buffer->LDS copies, one stage in flight per wave), the
    same with the nontemporal bit, an empty kernel of the launch shape, the
    same stages read as 4-row x 256-byte copies, the one-vector kernel's
    full-line copies (rows of 4 mod 8 blocks), and the lanes' operands loaded
    straight into registers with two stages in flight per wave (Q4_K).  The
    matvec cannot beat its own copy form's time."""
    out = {}
    per_graph = copies * max(1, GRAPH_CALLS // copies)
    reps = max(1, steps // per_graph)
    modes = [(0, "copies_us"), (1, "copies_nontemporal_us"), (2, "empty_launch_us"),
             (3, "copies_4x256_us")]
    if (cols // 256) % 8 == 4:  # Q4_K rows of 4 mod 8 blocks: the kernel's full-line copies
        modes.append((4, "copies_lines_us"))
    if ggml_type == 12:
        modes += [(5, "registers_2_in_flight_us"), (6, "registers_2_in_flight_nontemporal_us")]
    for mode, name in modes:
        # recorded into a HIP graph and replayed, so that host launch cost
        # does not pace the short launches
        ctx.capture_begin()
        rc = lib.si_hip_stream_probe(ctx.handle, harr, copies, rows, cols, mode, per_graph)
        graph = ctx.capture_end()
        if rc:
            graph.free()
            raise si_hip.HipError(rc, si_hip.last_error())
        for _ in range(max(1, warmup // per_graph)):
            graph.launch()
        ctx.synchronize()
        ctx.event_record(0)
        for _ in range(reps):
            graph.launch()
        ctx.event_record(1)
        us = ctx.event_elapsed_ms(0, 1) * 1000.0 / (reps * per_graph)
        ctx.synchronize()
        graph.free()
        out[name] = round(us, 3)
    for name in ("copies_us", "copies_lines_us", "registers_2_in_flight_us"):
        if name in out:
            out[name.replace("_us", "_frac_of_peak")] = round(
                nbytes / (out[name] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    out["note"] = ("si_hip_stream_probe: the matvec's weight copies without arithmetic, "
                   "back to back over the same resident copies, replayed from a HIP graph")
    return out


GRAPH_CALLS = int(os.environ.get("SI_BENCH_GRAPH_CALLS", "64"))


def time_graph_repeat(ctx, lib, harr, copies, rows, cols, d_x, d_y, steps: int,
                      warmup: int) -> float:
    """Average ms per matvec when GRAPH_CALLS calls (cycling through the
    resident copies) are recorded once into a HIP graph (si_hip_capture_begin/
    end) and the graph is replayed back to back: the launch overhead per kernel
    of a captured decode step rather than of separate host launches."""
    import ctypes as C
    ctx.capture_begin()
    per_graph = copies * max(1, GRAPH_CALLS // copies)
    rc = lib.si_hip_quant_matvec_device_repeat(ctx.handle, harr, copies, rows, cols,
                                               C.c_void_p(d_x), C.c_void_p(d_y), per_graph)
    graph = ctx.capture_end()
    if rc:
        graph.free()
        raise si_hip.HipError(rc, si_hip.last_error())
    reps = max(1, steps // per_graph)
    for _ in range(max(1, warmup // per_graph)):
        graph.launch()
    ctx.synchronize()
    ctx.event_record(0)
    for _ in range(reps):
        graph.launch()
    ctx.event_record(1)
    ms = ctx.event_elapsed_ms(0, 1)
    ctx.synchronize()
    graph.free()
    return ms / (reps * per_graph)


def call_detail(ctx, lib, harr, weights, rows, cols, x, d_x, d_y, samples: int,
                host_bytes=None) -> dict:
    """Per-call device time of isolated calls (events around each call, the
    stream drained in between: p10/p50/p90), and host wall time per call of
    the synchronous host-pointer API (x copied in through pinned staging, y
    copied out, one wait): on a retained weight, and on borrowed host bytes
    (q4_k_matvec) once they are resident in HBM."""
    import ctypes as C
    per = []
    copies = len(weights)
    for i in range(samples):
        one = (C.c_void_p * 1)(harr[i % copies])
        ctx.event_record(2)
        rc = lib.si_hip_quant_matvec_device_repeat(ctx.handle, one, 1, rows, cols,
                                                   C.c_void_p(d_x), C.c_void_p(d_y), 1)
        if rc:
            raise si_hip.HipError(rc, si_hip.last_error())
        ctx.event_record(3)
        ctx.synchronize()
        per.append(ctx.event_elapsed_ms(2, 3) * 1000.0)
    per = np.array(per)
    n_wall = max(20, samples // 2)
    for i in range(5):
        ctx.gguf_quant_matvec_weight(weights[i % copies], rows, cols, x)
    t0 = time.perf_counter()
    for i in range(n_wall):
        ctx.gguf_quant_matvec_weight(weights[i % copies], rows, cols, x)
    wall = (time.perf_counter() - t0) / n_wall * 1e6
    borrowed = {}
    if host_bytes is not None and host_bytes.size * 2 <= si_hip.DEFAULT_RESIDENCY_BUDGET:
        ctx.residency_evict()
        s0 = ctx.residency_stats()
        t0 = time.perf_counter()
        ctx.q4_k_matvec(host_bytes, rows, cols, x)  # first call: the bytes go to HBM
        first = (time.perf_counter() - t0) * 1e6
        for _ in range(5):
            ctx.q4_k_matvec(host_bytes, rows, cols, x)
        t0 = time.perf_counter()
        for _ in range(n_wall):
            ctx.q4_k_matvec(host_bytes, rows, cols, x)
        bw = (time.perf_counter() - t0) / n_wall * 1e6
        s1 = ctx.residency_stats()
        borrowed = {"borrowed_bytes_host_wall_us_per_call": round(bw, 2),
                    "borrowed_bytes_first_call_us": round(first, 1),
                    "borrowed_bytes_note": (
                        f"q4_k_matvec on host bytes: {s1['uploads'] - s0['uploads']} weight "
                        f"copy to HBM over {n_wall + 6} calls, {s1['hits'] - s0['hits']} "
                        "resident hits")}
        ctx.residency_evict()
    return {**borrowed, "isolated_call_us": {"p10": round(float(np.percentile(per, 10)), 3),
                                 "p50": round(float(np.percentile(per, 50)), 3),
                                 "p90": round(float(np.percentile(per, 90)), 3),
                                 "samples": samples},
            "host_wall_us_per_call": round(wall, 2),
            "host_wall_note": "synchronous C-ABI call on a retained weight with host x and "
                              "y (x through pinned staging, kernel, y back, stream wait), "
                              f"averaged over {n_wall} calls"}


def _timed(ctx, fn, steps: int, warmup: int, warm_ms: float = WARM_MS) -> float:
    """Average ms per call of fn(i) enqueued back to back on the compute stream,
    after at least `warmup` untimed calls and warm_ms of them (a GPU left idle
    by host work, e.g. weight uploads, clocks down and needs some 10 ms of
    calls to come back)."""
    t0 = time.perf_counter()
    i = 0
    while i < warmup or (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(25):
            fn(i)
            i += 1
        ctx.synchronize()
    ctx.event_record(0)
    for i in range(steps):
        fn(i)
    ctx.event_record(1)
    ms = ctx.event_elapsed_ms(0, 1)
    ctx.synchronize()
    return ms / steps


GRAPHS = True  # False (--no-graphs): no leg replays a HIP graph


def _timed_graph(ctx, fn, per_graph: int, steps: int, warmup: int) -> float | None:
    """Average ms per call of fn(i) when per_graph calls are recorded once
    into a HIP graph and the graph is replayed back to back: the device time
    of short calls without the Python and host launch cost of each call.
    None when graph legs are off."""
    if not GRAPHS:
        return None
    ctx.capture_begin()
    try:
        for i in range(per_graph):
            fn(i)
    finally:
        graph = ctx.capture_end()
    try:
        reps = max(1, steps // per_graph)
        for _ in range(max(1, warmup // per_graph)):
            graph.launch()
        ctx.synchronize()
        ctx.event_record(0)
        for _ in range(reps):
            graph.launch()
        ctx.event_record(1)
        ms = ctx.event_elapsed_ms(0, 1)
        ctx.synchronize()
    finally:
        graph.free()
    return ms / (reps * per_graph)


def _rate(nbytes: int, ms: float) -> dict:
    us = ms * 1000.0
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"bytes_per_call": nbytes, "us_per_call": round(us, 3), "gb_per_s": round(gbs, 1),
            "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4)}


CONFIG_NAMES = ("sweep", "mlp", "q5k", "head", "embedding", "many", "aggregate")
# (the aggregate uploads 10 GB of weights, a few seconds)
DEFAULT_CONFIGS = CONFIG_NAMES


def run_configs(ctx, steps: int, warmup: int, only=CONFIG_NAMES) -> dict:
    """BASELINE configs 2-5 on the HBM-resident device path (synthetic data);
    `only` picks some of CONFIG_NAMES."""
    import ctypes as C
    lib = si_hip.lib()
    Q4, Q5, Q6 = si_hip.GGML_TYPE_Q4_K, si_hip.GGML_TYPE_Q5_K, si_hip.GGML_TYPE_Q6_K
    res: dict = {}

    def upload(t, seed, rows, cols):
        w = si_hip.synth_matrix(t, seed=seed, rows=rows, cols=cols, threads=16)
        h = ctx.upload_quant_weight_private(w, t)
        del w
        return h

    def dev_f32(values):
        a = np.ascontiguousarray(values, dtype=np.float32)
        p = ctx.device_alloc(a.nbytes)
        ctx.to_device(p, a)
        return p

    def bpc(t, rows, cols):
        return rows * (cols // 256) * si_hip.BLOCK_BYTES[t]

    N, K = 17408, 5120
    if "sweep" in only:
        # config 2: the batch-1 Q4_K shapes other than the headline's
        sweep = {}
        for r, c in ((5120, 5120), (5120, 17408), (1024, 5120)):
            m = time_matvec(ctx, Q4, r, c, steps, warmup)
            log(f"configs: sweep {r}x{c}: {m['us_per_call']} us, {m['gb_per_s']} GB/s")
            sweep[f"{r}x{c}"] = {k: m[k] for k in ("bytes_per_call", "us_per_call", "gb_per_s",
                                                  "frac_of_peak", "weight_copies",
                                                  "resident_bytes")}
        res["q4k_sweep"] = sweep
    if "mlp" in only:
        res.update(_config_mlp(ctx, lib, upload, dev_f32, bpc, steps, warmup, N, K))
    if {"q5k", "head", "embedding"} & set(only):
        res.update(_config_mixed(ctx, lib, upload, dev_f32, bpc, steps, warmup, K, only))
    if "many" in only:
        res.update(_config_many(ctx, lib, upload, dev_f32, bpc, steps, warmup, N, K))
    if "aggregate" in only:
        res.update(_config_aggregate(ctx, lib, dev_f32, bpc))
    return res


def _config_mlp(ctx, lib, upload, dev_f32, bpc, steps, warmup, N, K) -> dict:
    import ctypes as C
    Q4, Q6 = si_hip.GGML_TYPE_Q4_K, si_hip.GGML_TYPE_Q6_K
    res = {}
    # config 3: fused SwiGLU (gate/up Q4_K 17408x5120, down Q6_K 5120x17408), 3 copies
    log("configs: fused SwiGLU MLP")
    mlp = [(upload(Q4, 300 + c, N, K), upload(Q4, 310 + c, N, K), upload(Q6, 320 + c, K, N))
           for c in range(3)]
    x = dev_f32(si_hip.synth_normal(301, K) * np.float32(0.1))
    h = ctx.device_alloc(N * 4)
    y = ctx.device_alloc(K * 4)
    gu_ms = _timed(ctx, lambda i: si_hip._check(lib.si_hip_q4_k_fused_gate_up_device(
        ctx.handle, mlp[i % 3][0].handle, mlp[i % 3][1].handle, N, K, C.c_void_p(x),
        C.c_void_p(h))), steps, warmup)
    mlp_ms = _timed(ctx, lambda i: si_hip._check(lib.si_hip_fused_mlp_device(
        ctx.handle, mlp[i % 3][0].handle, mlp[i % 3][1].handle, mlp[i % 3][2].handle, N, K, K,
        C.c_void_p(x), C.c_void_p(h), C.c_void_p(y))), steps, warmup)
    res["fused_gate_up_q4k_17408x5120"] = {**_rate(2 * bpc(Q4, N, K), gu_ms),
                                           **residency(2 * bpc(Q4, N, K), 3)}
    res["fused_mlp_q4k_gate_up_q6k_down"] = {
        **_rate(2 * bpc(Q4, N, K) + bpc(Q6, K, N), mlp_ms),
        **residency(2 * bpc(Q4, N, K) + bpc(Q6, K, N), 3)}
    for g, u, d in mlp:
        g.free(); u.free(); d.free()
    for p in (x, h, y):
        ctx.device_free(p)
    return res


def _config_mixed(ctx, lib, upload, dev_f32, bpc, steps, warmup, K, only) -> dict:
    import ctypes as C
    Q4, Q5, Q6 = si_hip.GGML_TYPE_Q4_K, si_hip.GGML_TYPE_Q5_K, si_hip.GGML_TYPE_Q6_K
    res = {}
    # config 4: Q5_K 5120x5120, Q6_K head 151936x5120 + argmax, Q4_K embedding of 64 ids
    log("configs: Q5_K matvec, Q6_K head + argmax, Q4_K embedding")
    x = dev_f32(si_hip.synth_normal(401, K))
    y = ctx.device_alloc(K * 4)
    if "q5k" in only:
        n5 = copies_for(bpc(Q5, K, K))
        q5 = [upload(Q5, 400 + c, K, K) for c in range(n5)]

        def q5_call(i):
            si_hip._check(lib.si_hip_quant_matvec_device(
                ctx.handle, q5[i % n5].handle, K, K, C.c_void_p(x), C.c_void_p(y)))

        res["q5k_matvec_5120x5120"] = {**_rate(bpc(Q5, K, K), _timed(ctx, q5_call, steps, warmup)),
                                       **residency(bpc(Q5, K, K), n5)}
        g = _timed_graph(ctx, q5_call, 64, steps, warmup)
        if g is not None:
            res["q5k_matvec_5120x5120"]["graph_us_per_call"] = round(1000.0 * g, 3)
        for w in q5:
            w.free()
    V = 151936
    if "head" in only:
        head = upload(Q6, 410, V, K)
        logits = ctx.device_alloc(V * 4)
        packed = ctx.device_alloc(8)
        ms = _timed(ctx, lambda i: si_hip._check(lib.si_hip_matvec_argmax_device(
            ctx.handle, head.handle, V, K, C.c_void_p(x), 0, C.c_void_p(logits),
            C.c_void_p(packed))), max(steps // 4, 10), max(warmup // 4, 2))
        res["q6k_head_argmax_151936x5120"] = {**_rate(bpc(Q6, V, K), ms),
                                              **residency(bpc(Q6, V, K), 1)}
        head.free()
        ctx.device_free(logits); ctx.device_free(packed)
    if "embedding" in only:
        table = upload(Q4, 420, V, K)
        # calls rotate through id sets of distinct rows (a seeded permutation
        # of the table's rows) that together exceed the MALL
        row_b = bpc(Q4, 1, K)
        nsets = min(V // 64, copies_for(64 * row_b))
        ids = ctx.device_alloc(nsets * 64 * 4)
        perm = np.random.default_rng(421).permutation(V)[:nsets * 64]
        ctx.to_device(ids, perm.astype(np.uint32))
        emb = ctx.device_alloc(64 * K * 4)
        def emb_call(i):
            si_hip._check(lib.si_hip_embedding_device(
                ctx.handle, table.handle, K, V, C.c_void_p(ids + 256 * (i % nsets)), 64,
                C.c_void_p(emb)))

        res["q4k_embedding_64_tokens"] = _rate(64 * row_b, _timed(ctx, emb_call, steps, warmup))
        res["q4k_embedding_64_tokens"].update(
            {"id_sets": nsets, "resident_bytes": nsets * 64 * row_b,
             "note": "each call 64 ids of a different set, every row of every set distinct"})
        g = _timed_graph(ctx, emb_call, 64, steps, warmup)
        if g is not None:
            res["q4k_embedding_64_tokens"]["graph_us_per_call"] = round(1000.0 * g, 3)
        table.free()
        ctx.device_free(ids); ctx.device_free(emb)
    for p in (x, y):
        ctx.device_free(p)
    return res


def _config_many(ctx, lib, upload, dev_f32, bpc, steps, warmup, N, K) -> dict:
    import ctypes as C
    Q4 = si_hip.GGML_TYPE_Q4_K
    res = {}
    # config 5: matmul-many M in {1,2,4,8,16} on Q4_K 17408x5120, 8 copies
    log("configs: multi-token verify")
    ws = [upload(Q4, 500 + c, N, K) for c in range(8)]
    X = dev_f32(si_hip.synth_normal(501, 16 * K))
    Y = ctx.device_alloc(16 * N * 4)
    many = {}
    for m in (1, 2, 4, 8, 16):
        ms = _timed(ctx, lambda i, m=m: si_hip._check(lib.si_hip_matmul_many_device(
            ctx.handle, ws[i % 8].handle, N, K, m, C.c_void_p(X), C.c_void_p(Y))), steps, warmup)
        r = _rate(bpc(Q4, N, K), ms)
        r["tflop_per_s"] = round(2.0 * m * N * K / (ms * 1e-3) / 1e12, 3)
        many[f"M{m}"] = r
    many.update(residency(bpc(Q4, N, K), 8))
    res["matmul_many_q4k_17408x5120"] = many
    for w in ws:
        w.free()
    ctx.device_free(X); ctx.device_free(Y)
    # the same verify on Q5_K 5120x5120 (BASELINE config 3's matrix)
    Q5, N5, K5 = si_hip.GGML_TYPE_Q5_K, 5120, 5120
    n5 = copies_for(bpc(Q5, N5, K5))
    w5 = [upload(Q5, 520 + c, N5, K5) for c in range(n5)]
    X5 = dev_f32(si_hip.synth_normal(521, 16 * K5))
    Y5 = ctx.device_alloc(16 * N5 * 4)
    many5 = {}
    for m in (1, 4, 8, 16):
        ms = _timed(ctx, lambda i, m=m: si_hip._check(lib.si_hip_matmul_many_device(
            ctx.handle, w5[i % n5].handle, N5, K5, m, C.c_void_p(X5), C.c_void_p(Y5))), steps, warmup)
        r = _rate(bpc(Q5, N5, K5), ms)
        r["tflop_per_s"] = round(2.0 * m * N5 * K5 / (ms * 1e-3) / 1e12, 3)
        many5[f"M{m}"] = r
    many5.update(residency(bpc(Q5, N5, K5), n5))
    res["matmul_many_q5k_5120x5120"] = many5
    for w in w5:
        w.free()
    ctx.device_free(X5); ctx.device_free(Y5)
    # grouped matvec over one x (q/k/v-like projections): one launch against
    # one launch per matrix
    g_rows = (6144, 1024, 1024)
    g_bytes = sum(bpc(Q4, r, K) for r in g_rows)
    ng = copies_for(g_bytes)
    gws = [[upload(Q4, 510 + 3 * c + i, r, K) for i, r in enumerate(g_rows)] for c in range(ng)]
    Xg = dev_f32(si_hip.synth_normal(511, K))
    Yg = ctx.device_alloc(sum(g_rows) * 4)
    g_handles = [(C.c_void_p * 3)(*[wq.handle.value for wq in grp]) for grp in gws]
    g_rarr = (C.c_size_t * 3)(*g_rows)

    def one_launch(i):
        si_hip._check(lib.si_hip_quant_matvec_many_device(ctx.handle, g_handles[i % ng], g_rarr, 3,
                                                          K, C.c_void_p(Xg), C.c_void_p(Yg)))

    ms_one = _timed(ctx, one_launch, steps, warmup)
    ms_one_graph = _timed_graph(ctx, one_launch, 64, steps, warmup)

    def per_matrix(i):
        off = 0
        for wq, r in zip(gws[i % ng], g_rows):
            si_hip._check(lib.si_hip_quant_matvec_device(ctx.handle, wq.handle, r, K,
                                                         C.c_void_p(Xg), C.c_void_p(Yg + 4 * off)))
            off += r

    ms_each = _timed(ctx, per_matrix, steps, warmup)
    res["grouped_q4k_6144+1024+1024x5120"] = {
        "bytes_per_call": g_bytes, "one_launch": _rate(g_bytes, ms_one),
        "launch_per_matrix": _rate(g_bytes, ms_each), **residency(g_bytes, ng)}
    if ms_one_graph is not None:
        res["grouped_q4k_6144+1024+1024x5120"]["one_launch"]["graph_us_per_call"] = round(
            1000.0 * ms_one_graph, 3)
    for grp in gws:
        for wq in grp:
            wq.free()
    ctx.device_free(Xg); ctx.device_free(Yg)
    # the same verify through the Q6_K output head (638 MB, one copy: it
    # exceeds the 256 MB MALL on its own)
    Q6, HN = si_hip.GGML_TYPE_Q6_K, 151936
    head = upload(Q6, 502, HN, K)
    X = dev_f32(si_hip.synth_normal(503, 16 * K))
    Y = ctx.device_alloc(16 * HN * 4)
    many = {}
    for m in (1, 4, 8, 16):
        ms = _timed(ctx, lambda i, m=m: si_hip._check(lib.si_hip_matmul_many_device(
            ctx.handle, head.handle, HN, K, m, C.c_void_p(X), C.c_void_p(Y))),
            max(4, steps // 4), min(warmup, 2))
        r = _rate(bpc(Q6, HN, K), ms)
        r["tflop_per_s"] = round(2.0 * m * HN * K / (ms * 1e-3) / 1e12, 3)
        many[f"M{m}"] = r
    many.update(residency(bpc(Q6, HN, K), 1))
    res["matmul_many_q6k_head_151936x5120"] = many
    head.free()
    ctx.device_free(X); ctx.device_free(Y)
    return res


def _config_aggregate(ctx, lib, dev_f32, bpc) -> dict:
    import ctypes as C
    Q4, Q6 = si_hip.GGML_TYPE_Q4_K, si_hip.GGML_TYPE_Q6_K
    res = {}
    # config 5b: 64 synthetic 27B-class layers streamed once per token
    log("configs: 64-layer aggregate")
    layer_shapes = [(Q4, 16384, 5120), (Q4, 5120, 6144), (Q4, 17408, 5120), (Q4, 17408, 5120),
                    (Q6, 5120, 17408)]
    host = [si_hip.synth_matrix(t, seed=600 + i, rows=r, cols=c, threads=16)
            for i, (t, r, c) in enumerate(layer_shapes)]
    layers = [[ctx.upload_quant_weight_private(hb, t) for hb, (t, _, _) in zip(host, layer_shapes)]
              for _ in range(64)]
    del host
    xin = dev_f32(si_hip.synth_normal(601, 17408))
    ybuf = ctx.device_alloc(17408 * 4)
    hbuf = ctx.device_alloc(17408 * 4)
    layer_bytes = sum(bpc(t, r, c) for t, r, c in layer_shapes)

    def token(_i):
        for L in layers:
            si_hip._check(lib.si_hip_quant_matvec_device(ctx.handle, L[0].handle, 16384, 5120,
                                                         C.c_void_p(xin), C.c_void_p(ybuf)))
            si_hip._check(lib.si_hip_quant_matvec_device(ctx.handle, L[1].handle, 5120, 6144,
                                                         C.c_void_p(xin), C.c_void_p(ybuf)))
            si_hip._check(lib.si_hip_fused_mlp_device(ctx.handle, L[2].handle, L[3].handle,
                                                      L[4].handle, 17408, 5120, 5120,
                                                      C.c_void_p(xin), C.c_void_p(hbuf),
                                                      C.c_void_p(ybuf)))
    ms = _timed(ctx, token, 5, 1)
    agg = _rate(64 * layer_bytes, ms)
    agg["ms_per_token"] = round(ms, 3)
    agg["tb_per_s"] = round(64 * layer_bytes / (ms * 1e-3) / 1e12, 3)
    agg.update(residency(64 * layer_bytes, 1))
    agg["layers"] = 64
    agg["per_layer"] = "qkv Q4_K 16384x5120, o Q4_K 5120x6144, gate/up Q4_K 17408x5120 fused, down Q6_K 5120x17408"
    res["aggregate_64_layers"] = agg
    for L in layers:
        for w in L:
            w.free()
    for p in (xin, ybuf, hbuf):
        ctx.device_free(p)
    return res


def profiled_traffic() -> int | None:
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_baseline(rows: int, cols: int, budget_s: float = 10.0, threads: int = 1) -> dict:
    """Reference CPU path (oracle restatement of quant.rs + host dot) on
    `threads` host threads (rows split between them; results identical)."""
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
        rc = lib.kq_matvec_ref(12, bp, w.size, rows, cols, xp, yp, None, None, threads)
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
    return {"value": round(w.size / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_call": round(dt * 1e6, 1),
            "sample": f"{calls} full Q4_K {rows}x{cols} calls (quant.rs dequant + sequential f32 "
                      f"dot), oracle/kquant_ref.c -O2 -ffp-contract=off, {model}"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # (from an idle start the headline matvec needs about a thousand calls,
    # some 13 ms, to reach its steady rate: the first hundred run ~6% slower)
    ap.add_argument("--warmup", type=int, default=2000,
                    help="untimed calls before each timed headline leg (the configs, timed "
                         "after the headline on a warm GPU, take at most 100)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--configs", nargs="?", const=",".join(CONFIG_NAMES),
                    default=",".join(DEFAULT_CONFIGS),
                    help="BASELINE configs 2-5 timed after the headline: a comma list of "
                         f"{','.join(CONFIG_NAMES)} (default: {','.join(DEFAULT_CONFIGS)}; "
                         "the flag alone: all)")
    ap.add_argument("--no-configs", action="store_true", help="time the headline only")
    ap.add_argument("--back-to-back-only", action="store_true",
                    help="time the headline's back-to-back calls alone (no graph, isolated, "
                         "host-call or floor legs), for a kernel trace of exactly those calls")
    ap.add_argument("--no-graphs", action="store_true",
                    help="skip every leg that replays a HIP graph (for profiler runs: "
                         "rocprofv3's kernel trace has crashed in a graph launch)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also time device-to-device copies of the matrix size (the yardstick "
                         "that scales HBM traffic counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the matvec "
              "would shard its rows across GPUs, each streaming its share of the weights)",
              file=sys.stderr)
        return 2

    ctx = si_hip.HipContext(0)
    rows, cols = 17408, 5120
    log(f"timing Q4_K {rows}x{cols}, {args.steps} steps, {NCOPIES} resident copies")
    b2b = args.back_to_back_only
    global GRAPHS
    GRAPHS = not args.no_graphs
    head = time_matvec(ctx, 12, rows, cols, args.steps, args.warmup, copies=NCOPIES,
                       detail=not b2b, graph=GRAPHS and not b2b)
    log(f"  {head['us_per_call']} us/call, {head['gb_per_s']} GB/s")
    out = {
        "metric": METRIC,
        "value": head["gb_per_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_done": {"calls": head["warmup_calls"], "ms": head["warmup_ms"],
                        "note": f"at least --warmup calls and {WARM_MS:g} ms of them"},
        "ms_per_step": round(head["us_per_call"] / 1000.0, 6),
        "us_per_call": head["us_per_call"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("q4_k weights (u8 packed; 4-bit quants, 6-bit scales) x activations as "
                  "block fixed point (per 256-element block: an exponent and 30-bit integers "
                  "in four int8 digits; tiny or non-finite elements exact in f32), int8 MFMA "
                  "with int32 accumulate, f32 combine of block sums"),
        "data": "synthetic (seeded generator, BASELINE.json config 2)",
        "config": {"workload": "Q4_K matvec N=17408 x K=5120, batch 1", "rows": rows,
                   "cols": cols, "batch": 1, "weight_copies": NCOPIES,
                   "resident_bytes": head["resident_bytes"],
                   "bytes_per_call": head["bytes_per_call"]},
        "roofline": {"bound": "hbm", "achieved": head["gb_per_s"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": head["frac_of_peak"],
                     "traffic": profiled_traffic()},
    }
    for k in ("graph_us_per_call", "graph_gb_per_s", "isolated_call_us", "host_wall_us_per_call",
              "host_wall_note", "floor", "borrowed_bytes_host_wall_us_per_call",
              "borrowed_bytes_first_call_us", "borrowed_bytes_note"):
        if k in head:
            out[k] = head[k]
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
    if args.configs and not args.no_configs:
        only = tuple(c for c in args.configs.split(",") if c)
        bad = [c for c in only if c not in CONFIG_NAMES]
        if bad:
            print(f"unknown config(s) {bad}; choose from {CONFIG_NAMES}", file=sys.stderr)
            return 2
        cfg_warmup = min(args.warmup, 100)
        out["configs"] = run_configs(ctx, args.steps, cfg_warmup, only)
        # config 1: the matrix the reference's CPU path is quoted on
        c1 = time_matvec(ctx, 12, 4096, 5120, args.steps, cfg_warmup)
        out["configs"]["q4k_matvec_4096x5120"] = {k: c1[k] for k in (
            "bytes_per_call", "us_per_call", "gb_per_s", "frac_of_peak", "weight_copies",
            "resident_bytes")}
    ctx.close()
    if not args.no_cpu:
        log("timing the CPU baseline")
        out["cpu_baseline"] = cpu_baseline(rows, cols, args.cpu_seconds)
        # all host cores the box gives this process (rows split between threads)
        cores = min(int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)),
                    os.cpu_count() or 1, 64)
        log(f"timing the CPU baseline on {cores} threads")
        out["cpu_baseline_all_cores"] = cpu_baseline(rows, cols, args.cpu_seconds, threads=cores)
        log("timing the CPU baseline at config 1 (4096x5120)")
        out["cpu_baseline_config1"] = cpu_baseline(4096, 5120, args.cpu_seconds / 2)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
