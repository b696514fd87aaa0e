"""GPU: one context shared by two host threads, as the reference's runtime
shares its Metal context between staging workers that upload weights and the
thread that runs the forward pass (qwen35_runtime.rs:1818-1904; the upload
queue beside the compute queue, metal.rs:1784-1785; QuantWeight upload,
metal.rs:2585-2636).

One thread uploads weights (private and "mapped"), reads a sample of each
back, takes a view of it and frees it, in a loop; the other runs matvecs on
uploaded weights, fused MLPs, matmul-many and residency-backed byte calls on
the same context.  Bar: every output equals the same call's output in a
serial run bit for bit, both threads finish (no deadlock), and the context's
counters add up: the command counts of the concurrent run equal those of the
two workloads run one after the other, the residency counters show only hits,
and the allocated bytes return to where they started.
"""
import threading
import time

import numpy as np
import pytest

import si_hip

pytestmark = pytest.mark.gpu

Q4, Q5, Q6 = 12, 13, 14
COUNTS = ("submitted", "async_submitted", "waited")


def log(msg):
    print(msg, flush=True)


class Compute:
    """The compute thread's fixed sequence of calls on one context."""

    def __init__(self, ctx, rounds):
        self.ctx = ctx
        self.rounds = rounds
        n, k = 4096, 5120
        self.n, self.k = n, k
        self.mat = si_hip.synth_matrix(Q4, seed=9100, rows=n, cols=k, threads=8)
        self.bytes_w = si_hip.synth_matrix(Q5, seed=9101, rows=1024, cols=k, threads=8)
        self.W = ctx.upload_quant_weight_private(self.mat, Q4)
        self.G = ctx.upload_quant_weight_private(
            si_hip.synth_matrix(Q4, seed=9102, rows=n, cols=k, threads=8), Q4)
        self.U = ctx.upload_quant_weight_private(
            si_hip.synth_matrix(Q4, seed=9103, rows=n, cols=k, threads=8), Q4)
        self.D = ctx.upload_quant_weight_private(
            si_hip.synth_matrix(Q6, seed=9104, rows=k, cols=n, threads=8), Q6)
        self.xs = [si_hip.synth_normal(9200 + i, k, scale=0.5) for i in range(rounds)]
        self.X4 = np.stack([si_hip.synth_normal(9300 + b, k) for b in range(4)])

    def run(self):
        c, n, k = self.ctx, self.n, self.k
        out = []
        for x in self.xs:
            out.append(c.gguf_quant_matvec_weight(self.W, n, k, x))
            out.append(c.gguf_quant_fused_mlp_weights(self.G, self.U, self.D, n, k, k, x))
            out.append(c.q5_k_matvec(self.bytes_w, 1024, k, x))          # residency-backed
            out.append(c.gguf_quant_matvec_bytes(Q4, self.mat, n, k, x))  # residency-backed
            out.append(np.concatenate(c.gguf_quant_matmul_many_weight(self.W, n, k, 4, self.X4)))
        return out

    def free(self):
        for h in (self.W, self.G, self.U, self.D):
            h.free()


class Uploads:
    """The upload thread's loop: upload, read back a sample, view, free."""

    def __init__(self, ctx, iters):
        self.ctx = ctx
        specs = [(Q4, 2048, 5120), (Q6, 1024, 4096), (Q5, 512, 2304), (Q4, 8192, 5120)]
        self.items = []
        for i in range(iters):
            t, r, c = specs[i % len(specs)]
            self.items.append((t, r, c, i % 3 == 2,
                               si_hip.synth_matrix(t, seed=9400 + i, rows=r, cols=c, threads=8)))

    def run(self):
        ctx = self.ctx
        for t, rows, cols, mapped, raw in self.items:
            W = (ctx.bind_quant_weight_mapped(raw, t) if mapped
                 else ctx.upload_quant_weight_private(raw, t))
            try:
                assert W.byte_len() == raw.size and W.ggml_type() == t
                head = ctx.from_device(W.device_ptr(), (4096,), np.uint8)
                tail = ctx.from_device(W.device_ptr() + raw.size - 4096, (4096,), np.uint8)
                assert np.array_equal(head, raw[:4096]) and np.array_equal(tail, raw[-4096:])
                rb = raw.size // rows
                V = W.view(rb, rb, t)  # row 1
                try:
                    row1 = ctx.from_device(V.device_ptr(), (rb,), np.uint8)
                    assert np.array_equal(row1, raw[rb:2 * rb])
                finally:
                    V.free()
            finally:
                W.free()


def _stats(ctx):
    s = ctx.command_stats()
    r = ctx.residency_stats()
    return {**{k: s[k] for k in COUNTS}, **{k: r[k] for k in ("hits", "uploads", "evictions")},
            "allocated": ctx.current_allocated_bytes()}


def _delta(a, b):
    return {k: b[k] - a[k] for k in a}


def _run_threads(fns, timeout):
    """Runs the functions in threads started together; checks that all finish
    within `timeout` seconds and that their runs overlap in time."""
    errors, results, spans = [], {}, {}
    go = threading.Barrier(len(fns))

    def wrap(name, fn):
        try:
            go.wait()
            t0 = time.monotonic()
            results[name] = fn()
            spans[name] = (t0, time.monotonic())
        except BaseException as e:  # noqa: BLE001 - reported to the main thread
            errors.append((name, e))

    ts = [threading.Thread(target=wrap, args=(name, fn), daemon=True) for name, fn in fns]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout)
    stuck = [name for (name, _), t in zip(fns, ts) if t.is_alive()]
    assert not stuck, f"threads did not finish within {timeout} s: {stuck}"
    if errors:
        raise errors[0][1]
    assert max(a for a, _ in spans.values()) < min(b for _, b in spans.values()), spans
    return results


def test_upload_thread_beside_compute_thread():
    ctx = si_hip.HipContext(0)
    try:
        ctx.set_residency_budget(si_hip.DEFAULT_RESIDENCY_BUDGET)
        comp = Compute(ctx, rounds=12)
        up = Uploads(ctx, iters=48)
        log("serial compute (warm: resident ranges, staging sizes)")
        comp.run()
        up.run()
        s0 = _stats(ctx)
        log("serial compute")
        serial = comp.run()
        s1 = _stats(ctx)
        log("serial uploads")
        up.run()
        s2 = _stats(ctx)
        d_comp, d_up = _delta(s0, s1), _delta(s1, s2)
        assert d_comp["uploads"] == 0 and d_comp["hits"] == 2 * comp.rounds
        assert d_up["hits"] == d_up["uploads"] == 0
        assert d_comp["allocated"] == d_up["allocated"] == 0
        for rep in range(3):
            log(f"concurrent run {rep}")
            res = _run_threads([("compute", comp.run), ("uploads", up.run)], timeout=90)
            s3 = _stats(ctx)
            d = _delta(s2, s3)
            for k in COUNTS + ("hits", "uploads", "evictions", "allocated"):
                assert d[k] == d_comp[k] + d_up[k], (k, d, d_comp, d_up)
            conc = res["compute"]
            assert len(conc) == len(serial)
            for i, (a, b) in enumerate(zip(serial, conc)):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"output {i} differs"
            s2 = s3
        comp.free()
    finally:
        ctx.close()


def test_two_compute_threads_share_a_context():
    """Two threads each run the compute sequence on one context: the calls
    serialise, and each thread's outputs equal its serial ones."""
    ctx = si_hip.HipContext(0)
    try:
        a = Compute(ctx, rounds=6)
        b = Compute(ctx, rounds=6)
        b.xs = [x[::-1].copy() for x in b.xs]
        log("serial compute, two sequences")
        ra, rb = a.run(), b.run()
        s0 = _stats(ctx)
        ra, rb = a.run(), b.run()
        d_serial = _delta(s0, _stats(ctx))
        s1 = _stats(ctx)
        log("two compute threads")
        res = _run_threads([("a", a.run), ("b", b.run)], timeout=90)
        d = _delta(s1, _stats(ctx))
        assert {k: d[k] for k in COUNTS} == {k: d_serial[k] for k in COUNTS}
        for ser, conc in ((ra, res["a"]), (rb, res["b"])):
            for i, (x, y) in enumerate(zip(ser, conc)):
                assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), f"output {i}"
        a.free()
        b.free()
    finally:
        ctx.close()
