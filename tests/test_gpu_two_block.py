"""GPU: Q4_K and Q5_K matvecs in two-block stages.

A one-vector Q4_K / Q5_K launch moves four blocks of a 16-row tile per
(tile, stage) pair.  Where that leaves waves of a workgroup idle (Q4_K: fewer
pairs per workgroup than waves, and the two-block launch needs at most two
rounds), where 12 waves of four-block stages do not fit the LDS (Q4_K rows of
43 to 56 blocks), and for Q5_K whenever 12 waves fit, a stage holds two
blocks instead: 18 (Q4_K) or 22 (Q5_K) 16-byte pieces per row, copied as 5
or 6 copies of 4 pieces whose spare lanes re-read the row's last piece.  An
odd block count ends in a stage of one live block whose second block is the
next row's first (zeros past the tile's last row).

Bar: every row within 2e-5 * sum|w*x| of the f64 dot, +-inf / NaN rows
where per-weight f32 products give them, and the same bits on every call.
"""
import sys

import numpy as np
import pytest

import oracle_lib as O
import si_hip
from test_gpu_parity import _category, assert_dot_close, same_bits

pytestmark = pytest.mark.gpu

Q4, Q5 = 12, 13


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# (type, rows, cols): 16 blocks over 256 tiles; 21 blocks (odd) over a
# partial last tile; the 8192-row q/k/v-class shape; 56 blocks, where 12
# waves of four-block stages do not fit; 43 blocks (odd, no four-block fit);
# one partial tile of 9 blocks; Q5_K at 5120 x 5120, 21 blocks, an odd row
# count, the BASELINE gate shape (a split launch) and 68 blocks
SHAPES = [(Q4, 4096, 4096), (Q4, 1000, 5376), (Q4, 8192, 5120), (Q4, 4096, 14336),
          (Q4, 4096, 11008), (Q4, 17, 2304), (Q5, 5120, 5120), (Q5, 1000, 5376),
          (Q5, 4097, 2304), (Q5, 17408, 5120), (Q5, 5120, 17408)]


@pytest.mark.parametrize("t,rows,cols", SHAPES)
def test_two_block_within_tolerance(hip_ctx, t, rows, cols):
    log(f"two-block type {t} {rows}x{cols}")
    w = si_hip.synth_matrix(t, seed=rows * 3 + cols + t, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(rows + 5 * cols + t, cols)
    _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, t)
    try:
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        worst = assert_dot_close(y, y64, ab, what=f"type {t} {rows}x{cols}")
        log(f"  worst error / bound = {worst:.4f}")
        assert same_bits(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y)
    finally:
        W.free()


@pytest.mark.parametrize("t", [Q4, Q5])
def test_two_block_special_activations(hip_ctx, t):
    """Huge, side, subnormal and zero blocks in different stages of a 9-block
    row (the last stage holds one live block), then one infinite or NaN
    activation at a time, the last in the odd block."""
    rows, cols = 64, 2304
    w = si_hip.synth_matrix(t, seed=4700 + t, rows=rows, cols=cols, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, t)
    base = si_hip.synth_normal(4701, cols)
    try:
        x = base.copy()
        x[100:140] = np.float32(3e30)
        x[512 + 7] = np.float32(1e-9)
        x[512 + 300:512 + 303] = np.float32(-2e-10)
        x[1024:1280] = np.float32(1e-41)
        x[2048:2304] = 0.0
        _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
        assert_dot_close(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y64, ab,
                         what="special blocks")
        x = base.copy()
        x[2048:2304] = np.float32(-7e29)  # the odd block alone carries the huge values
        _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
        assert_dot_close(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y64, ab,
                         what="huge odd block")
        for k, v in [(3, np.inf), (700, -np.inf), (1500, np.nan), (2303, np.inf)]:
            x = base.copy()
            x[k] = v
            y32, _, _ = O.matvec(t, w, rows, cols, x, threads=8)
            y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
            assert np.array_equal(_category(y), _category(y32)), f"x[{k}] = {v}"
    finally:
        W.free()


def test_two_block_q5_k_matmul_many_and_one_vector(hip_ctx):
    """Five Q5_K vectors of an odd block count (21) in one vectors-in-rows
    pass (two groups, the second holding one vector), each within its bound
    and the same bits on a second call; a batch of one goes through the
    one-vector dispatch (two-block stages) and equals the plain matvec bit
    for bit."""
    rows, cols, batch = 1000, 5376, 5
    w = si_hip.synth_matrix(Q5, seed=4800, rows=rows, cols=cols, threads=8)
    X = si_hip.synth_normal(4801, batch * cols).reshape(batch, cols)
    W = hip_ctx.upload_quant_weight_private(w, Q5)
    try:
        outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
        again = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
        for b in range(batch):
            _, y64, ab = O.matvec(Q5, w, rows, cols, X[b], threads=8)
            assert_dot_close(outs[b], y64, ab, what=f"vector {b}")
            assert same_bits(outs[b], again[b])
        one = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, 1, X[4:5])
        assert same_bits(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, X[4]), one[0])
    finally:
        W.free()


def test_two_block_launches_in_a_graph(hip_ctx):
    """Two-block Q4_K and Q5_K launches (the Q5_K one split across
    workgroups) beside a four-block split Q4_K launch, recorded in one HIP
    graph and replayed three times with eager launches on the same workspace
    between the replays: every replay equals the eager run bit for bit."""
    import ctypes as C
    lib = si_hip.lib()
    P = C.c_void_p
    shapes = [(Q4, 4096, 4096), (Q5, 17408, 5120), (Q4, 17408, 5120), (Q5, 1000, 5376)]
    mats, ins, outs = [], [], []
    for t, rows, cols in shapes:
        w = si_hip.synth_matrix(t, seed=rows + cols + 11 * t, rows=rows, cols=cols, threads=8)
        mats.append((w, hip_ctx.upload_quant_weight_private(w, t)))
        x = si_hip.synth_normal(rows * 7 + cols, cols)
        d_x = hip_ctx.device_alloc(cols * 4)
        hip_ctx.to_device(d_x, x)
        ins.append((x, d_x))
        outs.append(hip_ctx.device_alloc(rows * 4))
    d_e = hip_ctx.device_alloc(17408 * 4)
    h = hip_ctx.handle

    def enqueue():
        for (t, rows, cols), (_, W), (_, d_x), d_y in zip(shapes, mats, ins, outs):
            rc = lib.si_hip_quant_matvec_device(h, W.handle, rows, cols, P(d_x), P(d_y))
            assert rc == 0, si_hip.last_error()

    def results():
        hip_ctx.synchronize()
        return [hip_ctx.from_device(d_y, rows) for (_, rows, _), d_y in zip(shapes, outs)]

    def clear():
        for (_, rows, _), d_y in zip(shapes, outs):
            hip_ctx.to_device(d_y, np.full(rows, np.nan, np.float32))

    try:
        enqueue()
        ref = results()
        for (t, rows, cols), (w, _), (x, _), y in zip(shapes, mats, ins, ref):
            _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
            assert_dot_close(y, y64, ab, what=f"eager type {t} {rows}x{cols}")
        log("two-block graph: capture")
        hip_ctx.capture_begin()
        enqueue()
        graph = hip_ctx.capture_end()
        try:
            for rep in range(3):
                clear()
                for k in (1, 2):
                    (t, rows, cols), (_, W), (_, d_x) = shapes[k], mats[k], ins[k]
                    assert lib.si_hip_quant_matvec_device(h, W.handle, rows, cols, P(d_x),
                                                          P(d_e)) == 0
                hip_ctx.synchronize()
                log(f"two-block graph replay {rep}")
                graph.launch()
                for a, b in zip(results(), ref):
                    assert same_bits(a, b), f"replay {rep} differs"
        finally:
            graph.free()
    finally:
        for _, W in mats:
            W.free()
        for _, d_x in ins:
            hip_ctx.device_free(d_x)
        for d_y in outs:
            hip_ctx.device_free(d_y)
        hip_ctx.device_free(d_e)


@pytest.mark.parametrize("seed", range(10))
def test_random_short_and_mid_rows(hip_ctx, seed):
    """Seeded random Q4_K / Q5_K shapes of 1 to 56 blocks (odd and even) and
    1 to 20000 rows: one-vector matvecs that land on two-block, four-block,
    split and sliced launches, every row within the oracle's bound and
    repeating its own bits."""
    rng = np.random.default_rng(9900 + seed)
    t = int(rng.choice([Q4, Q5]))
    cols = 256 * int(rng.choice([1, 2, 9, 16, 20, 21, 32, 43, 48, 56]))
    rows = int(rng.integers(1, 20000))
    log(f"random short/mid seed={seed}: type {t} {rows}x{cols}")
    w = si_hip.synth_matrix(t, seed=9950 + seed, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(9970 + seed, cols)
    W = hip_ctx.upload_quant_weight_private(w, t)
    try:
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
        assert_dot_close(y, y64, ab, what=f"type {t} {rows}x{cols}")
        assert same_bits(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y)
    finally:
        W.free()
