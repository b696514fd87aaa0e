"""GPU: weights that cancel inside their own decode, and the device argmax of
a head with no candidate.

Q4_K / Q5_K matrices from tests/cancel_blocks.py (rows where every weight is
exactly 0 because d * sc * q* == dmin * m, rows where 99 % or 90 % of them
are, and ordinary rows) through every launch form that computes the factored
dot d * sum(sc q X) - dmin * sum(m X): one vector (four-block, two-block and
K-sliced launches), the fused gate/up, the fused MLP, matmul-many (two to
sixteen vectors) and the grouped launch, under the default (matrix-core) and
the generic kernel policy.  Bar: every dot within 2e-5 * sum|w*x| of the f64
value of the exact products (quant.rs:45-59 per-weight values,
metal.rs:7478-7484 dot), so a row whose weights are all 0 must come out
exactly 0, as the reference's does.

The device head argmax (si_hip_matvec_argmax_device) of an all-NaN and an
all -inf head: si_hip_argmax_result_index gives 0 under the strict '>' rule,
the id qwen35_runtime.rs:2237-2244 keeps when no logit beats -inf, and
SI_HIP_ARGMAX_NONE under the finite-only rule, whose host call fails with
"logits contain no finite values" (runtime.rs:4301-4309).
"""
import ctypes as C
import sys

import numpy as np
import pytest

import cancel_blocks as CB
import oracle_lib as O
import si_hip
from test_gpu_parity import POLICIES, assert_dot_close, gate_up_bound, silu64

pytestmark = pytest.mark.gpu

Q4, Q5, Q6 = 12, 13, 14


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(params=POLICIES, ids=["auto", "generic"])
def ctx(request, hip_ctx):
    hip_ctx.set_kernel_policy(request.param)
    yield hip_ctx
    hip_ctx.set_kernel_policy(si_hip.KERNEL_AUTO)


def _x(seed, cols, scale=1.0):
    return si_hip.synth_normal(seed, cols, scale=scale)


def _check_rows(y, y64, ab, rows, what):
    kinds = CB.row_kinds(rows)
    assert np.all(y[(kinds == 0)] == 0.0), f"{what}: a fully cancelling row is not 0"
    return assert_dot_close(y, y64, ab, what=what)


# (type, rows, cols): four-block stages (17408 x 5120), two-block stages
# (5120 x 5120, 1024 x 5120), K slices (640 x 17408, 5120 x 17408)
SHAPES = [(Q4, 17408, 5120), (Q4, 5120, 5120), (Q4, 1024, 5120), (Q4, 640, 17408),
          (Q4, 5120, 17408), (Q5, 5120, 5120), (Q5, 1024, 17408)]


@pytest.mark.parametrize("t,rows,cols", SHAPES)
def test_cancelling_matvec(ctx, t, rows, cols):
    log(f"cancelling matvec type {t} {rows}x{cols}")
    w = CB.matrix(t, rows, cols, seed=rows + cols + t)
    x = _x(rows ^ cols, cols)
    _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
    W = ctx.upload_quant_weight_private(w, t)
    try:
        y = ctx.gguf_quant_matvec_weight(W, rows, cols, x)
    finally:
        W.free()
    worst = _check_rows(y, y64, ab, rows, f"type {t} {rows}x{cols}")
    log(f"  worst {worst:.4f} of the bar")


def test_cancelling_fused_gate_up(ctx):
    rows, cols = 17408, 5120
    log("cancelling fused gate/up 17408x5120")
    gw = CB.matrix(Q4, rows, cols, seed=71)
    uw = CB.matrix(Q4, rows, cols, seed=72)
    x = _x(73, cols, scale=0.1)
    _, g64, ag = O.matvec(Q4, gw, rows, cols, x, threads=16)
    _, u64, au = O.matvec(Q4, uw, rows, cols, x, threads=16)
    G = ctx.upload_quant_weight_private(gw, Q4)
    U = ctx.upload_quant_weight_private(uw, Q4)
    try:
        h = ctx.q4_k_fused_gate_up_weights(G, U, rows, cols, x)
    finally:
        G.free()
        U.free()
    h64 = silu64(g64) * u64
    bound = gate_up_bound(g64, ag, u64, au)
    ratio = np.abs(h - h64) / bound
    log(f"  worst {ratio.max():.4f} of the bound")
    assert np.all(ratio <= 1.0)
    assert np.all(h[CB.row_kinds(rows) == 0] == 0.0)


def test_cancelling_fused_mlp(ctx):
    n, k = 4096, 5120
    log("cancelling fused MLP 4096x5120 -> 5120x4096")
    gw = CB.matrix(Q4, n, k, seed=81)
    uw = CB.matrix(Q4, n, k, seed=82)
    dw = si_hip.synth_matrix(Q6, seed=83, rows=k, cols=n, threads=16)
    x = _x(84, k, scale=0.1)
    _, g64, ag = O.matvec(Q4, gw, n, k, x, threads=16)
    _, u64, au = O.matvec(Q4, uw, n, k, x, threads=16)
    h64 = silu64(g64) * u64
    hb = gate_up_bound(g64, ag, u64, au)
    wd = O.dequantize(Q6, dw, k * n).reshape(k, n).astype(np.float64)
    y64 = wd @ h64
    awd = np.abs(wd)
    bound = 2e-5 * (awd @ np.abs(h64)) + awd @ hb + 1e-30
    G = ctx.upload_quant_weight_private(gw, Q4)
    U = ctx.upload_quant_weight_private(uw, Q4)
    D = ctx.upload_quant_weight_private(dw, Q6)
    try:
        y = ctx.gguf_quant_fused_mlp_weights(G, U, D, n, k, k, x)
    finally:
        for h in (G, U, D):
            h.free()
    ratio = np.abs(y - y64) / bound
    log(f"  worst {ratio.max():.4f} of the bound")
    assert np.all(ratio <= 1.0)


@pytest.mark.parametrize("t,batch", [(Q4, 2), (Q4, 4), (Q4, 8), (Q4, 13), (Q4, 16), (Q5, 4), (Q5, 8),
                                     (Q5, 16)])
def test_cancelling_matmul_many(ctx, t, batch):
    rows, cols = 4096, 5120
    log(f"cancelling matmul-many type {t} M={batch}")
    w = CB.matrix(t, rows, cols, seed=90 + batch + t)
    X = np.stack([_x(900 + b, cols) for b in range(batch)])
    W = ctx.upload_quant_weight_private(w, t)
    try:
        ys = ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    finally:
        W.free()
    for b in range(batch):
        _, y64, ab = O.matvec(t, w, rows, cols, X[b], threads=16)
        _check_rows(ys[b], y64, ab, rows, f"type {t} M={batch} vector {b}")


def test_cancelling_matmul_many_four_row_reduce(hip_ctx):
    # 33000 rows x 16 vectors: tok_reduce takes four rows a thread (528
    # workgroups of 1024 rows, the last one partial, and a partial last tile),
    # and the fully cancelling rows reach its exact recompute there
    t, rows, cols, batch = Q4, 33000, 5120, 16
    log(f"cancelling matmul-many type {t} {rows}x{cols} M={batch}")
    w = CB.matrix(t, rows, cols, seed=97)
    X = np.stack([_x(970 + b, cols) for b in range(batch)])
    W = hip_ctx.upload_quant_weight_private(w, t)
    try:
        ys = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    finally:
        W.free()
    for b in range(batch):
        _, y64, ab = O.matvec(t, w, rows, cols, X[b], threads=16)
        _check_rows(ys[b], y64, ab, rows, f"type {t} {rows} rows M={batch} vector {b}")


def test_cancelling_grouped(ctx):
    cols = 5120
    rows = [6144, 1024, 1024]
    log("cancelling grouped matvec 6144+1024+1024 x 5120")
    ws = [CB.matrix(Q4, r, cols, seed=100 + i) for i, r in enumerate(rows)]
    x = _x(110, cols)
    Ws = [ctx.upload_quant_weight_private(w, Q4) for w in ws]
    try:
        outs = ctx.gguf_quant_matvec_many_weights(Ws, rows, cols, x)
    finally:
        for W in Ws:
            W.free()
    for w, r, y in zip(ws, rows, outs):
        _, y64, ab = O.matvec(Q4, w, r, cols, x, threads=8)
        _check_rows(y, y64, ab, r, f"grouped {r}x{cols}")


# ---- the device head argmax with no candidate ----------------------------------
def _head_all_neg_inf(rows, cols):
    """Q6_K head whose element 0 decodes to -32 d sc < 0 in every row, so
    x[0] = +inf makes every logit -inf."""
    b = np.frombuffer(si_hip.synth_matrix(Q6, seed=7300, rows=rows, cols=cols).tobytes(),
                      np.uint8).reshape(rows, cols // 256, 210).copy()
    b[:, 0, 0] &= 0xF0          # ql[0] low nibble 0
    b[:, 0, 128] &= 0xFC        # qh[0] bits 0-1: q = 0
    b[:, 0, 192] = 5            # scale 0 > 0
    b[:, 0, 209] &= 0x7F        # d >= 0 (f16 sign bit clear) ...
    zero = (b[:, 0, 208] == 0) & (b[:, 0, 209] == 0)
    b[zero, 0, 209] = 0x3C      # ... and d = 1 where it was 0
    return b.tobytes()


def _device_head(hip_ctx, H, rows, cols, x, rule):
    lib = si_hip.lib()
    d_x = hip_ctx.device_alloc(cols * 4)
    d_l = hip_ctx.device_alloc(rows * 4)
    d_r = hip_ctx.device_alloc(8)
    try:
        hip_ctx.to_device(d_x, x)
        rc = lib.si_hip_matvec_argmax_device(hip_ctx.handle, H.handle, rows, cols,
                                             C.c_void_p(d_x), rule, C.c_void_p(d_l),
                                             C.c_void_p(d_r))
        if rc:
            raise si_hip.HipError(rc, si_hip.last_error())
        hip_ctx.synchronize()
        packed = int(hip_ctx.from_device(d_r, (1,), np.uint64)[0])
        logits = hip_ctx.from_device(d_l, (rows,))
    finally:
        for p in (d_x, d_l, d_r):
            hip_ctx.device_free(p)
    return packed, int(lib.si_hip_argmax_result_index(packed, rule)), logits


@pytest.mark.parametrize("policy", POLICIES, ids=["auto", "generic"])
@pytest.mark.parametrize("case", ["nan", "neg_inf"])
def test_device_argmax_without_candidate(hip_ctx, policy, case):
    rows, cols = 4099, 512
    x = si_hip.synth_normal(7301, cols)
    if case == "nan":
        w = si_hip.synth_matrix(Q6, seed=7302, rows=rows, cols=cols).tobytes()
        x[5] = np.nan
    else:
        w = _head_all_neg_inf(rows, cols)
        x[0] = np.inf
    log(f"device argmax, no candidate: {case}, policy {policy}")
    H = hip_ctx.upload_quant_weight_private(w, Q6)
    hip_ctx.set_kernel_policy(policy)
    try:
        packed, first, logits = _device_head(hip_ctx, H, rows, cols, x,
                                             si_hip.ARGMAX_FIRST_GREATER)
        if case == "nan":
            assert np.all(np.isnan(logits))
        else:
            assert np.all(logits == -np.inf)
        assert packed == 0
        assert first == 0 == O.argmax_first_greater(logits)
        packed, last, _ = _device_head(hip_ctx, H, rows, cols, x, si_hip.ARGMAX_LAST_FINITE)
        assert packed == 0 and last == 0xFFFFFFFF
        assert O.argmax_last_finite(logits) is None
        # the host calls: the strict rule keeps id 0, the finite-only one fails
        tok, _ = hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x,
                                                          rule=si_hip.ARGMAX_FIRST_GREATER)
        assert tok == 0
        with pytest.raises(si_hip.HipError) as e:
            hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x)
        assert e.value.status == -8
    finally:
        hip_ctx.set_kernel_policy(si_hip.KERNEL_AUTO)
        H.free()
