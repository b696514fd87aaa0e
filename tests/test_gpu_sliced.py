"""GPU: Q4_K, Q5_K and Q6_K matvecs of long rows over few tiles (down
projections), which run K-sliced: each workgroup takes one of S slices of
every tile's stages and holds only that slice's activation images, and a
tile's S slice sums meet in the workspace, added in slice order.

The launch takes four slices when an unsliced launch would give its busiest
workgroup at most 24 (tile, stage) pairs (K of 8192 or more) and slicing
takes some of them or the rows are long (64 blocks or more), and two or
four when the unsliced images would leave room for fewer than eight waves
and slicing adds no pairs; Q4_K and Q5_K rows longer than the unsliced
kernels take (more than 128 blocks) always slice.  (Q4_K / Q5_K shapes of
many tiles run two-block stages instead; test_gpu_two_block.py.)  The bar is the north
star's: every row within 2e-5 * sum|w*x| of the f64 dot, +-inf / NaN rows
where per-weight f32 products give them, and the same bits on every call.
"""
import sys

import numpy as np
import pytest

import oracle_lib as O
import si_hip
from test_gpu_parity import _category, assert_dot_close, same_bits

pytestmark = pytest.mark.gpu

Q4, Q5, Q6 = 12, 13, 14


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# (rows, cols): one tile (nb 48: four slices of 6 stages); a partial last
# tile and 25 stages (slices of 7, 6, 6, 6); 160 tiles of the down
# projection's K (three per workgroup, slices of 9, 9, 8, 8); 40 tiles (a
# tensor-parallel shard); the largest block count the unsliced kernel takes
# (128: two slices of 32 stages); one tile of 108 blocks; rows past 128
# blocks, which must slice (136 blocks: four slices of 17 stages; 256
# blocks: four of 32; 548 blocks: sixteen of 18)
SHAPES = [(16, 12288), (1000, 12800), (2560, 17408), (640, 17408), (2048, 32768), (3, 27648),
          (100, 34816), (2560, 34816), (40, 65536), (17, 140288)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_sliced_q6_k_within_tolerance(hip_ctx, rows, cols):
    log(f"sliced q6_k {rows}x{cols}")
    w = si_hip.synth_matrix(Q6, seed=rows * 7 + cols, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(rows + cols, cols)
    _, y64, ab = O.matvec(Q6, w, rows, cols, x, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, Q6)
    try:
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        worst = assert_dot_close(y, y64, ab, what=f"{rows}x{cols}")
        log(f"  worst error / bound = {worst:.4f}")
        # deterministic: the slices are added in slice order on every call
        assert same_bits(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y)
    finally:
        W.free()


# Q4_K / Q5_K: the BASELINE down shape (17 stages: slices of 5, 4, 4, 4);
# 136 blocks (past the unsliced kernels' 128); 129 blocks, odd, whose last
# slice ends in a partial stage; 13 stages over a partial last tile; the
# down shape's K over 64 tiles; one tile of 256 blocks (slices of 32
# blocks); 40 tiles; rows of 512 and 548 blocks over one tile (sixteen and
# thirty-two slices)
Q45_SHAPES = [(Q4, 5120, 17408), (Q4, 2560, 34816), (Q5, 100, 33024), (Q4, 1000, 12800),
              (Q5, 1024, 17408), (Q4, 3, 65536), (Q4, 640, 17408), (Q5, 640, 17408),
              (Q4, 3, 131072), (Q4, 16, 140288), (Q5, 16, 140288)]


@pytest.mark.parametrize("t,rows,cols", Q45_SHAPES)
def test_sliced_q4_q5_within_tolerance(hip_ctx, t, rows, cols):
    log(f"sliced type {t} {rows}x{cols}")
    w = si_hip.synth_matrix(t, seed=rows * 5 + cols + t, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(rows + cols + t, cols)
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
def test_sliced_q4_q5_special_activations(hip_ctx, t):
    """Huge, side, subnormal and zero blocks in different slices of a
    16384-column row, then one infinite or NaN activation at a time."""
    rows, cols = 200, 16384
    w = si_hip.synth_matrix(t, seed=4300 + t, rows=rows, cols=cols, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, t)
    base = si_hip.synth_normal(4301, cols)
    try:
        x = base.copy()
        x[100:140] = np.float32(3e30)
        x[4096 + 7] = np.float32(1e-9)
        x[4096 + 300:4096 + 303] = np.float32(-2e-10)
        x[8192:8192 + 256] = np.float32(1e-41)
        x[12288 + 512:12288 + 768] = 0.0
        _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
        assert_dot_close(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y64, ab,
                         what="special blocks")
        for k, v in [(50, np.inf), (4200, -np.inf), (9000, np.nan), (16383, np.inf)]:
            x = base.copy()
            x[k] = v
            y32, _, _ = O.matvec(t, w, rows, cols, x, threads=8)
            y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
            assert np.array_equal(_category(y), _category(y32)), f"x[{k}] = {v}"
    finally:
        W.free()


def test_sliced_special_activations_in_every_slice(hip_ctx):
    """Each slice of a 16384-column row (32 stages, 8 per slice) holds one
    kind of special block: huge values (fixed point would overflow), side
    elements (tiny next to their block's maximum), subnormals, zeros; then one
    infinite or NaN activation in one slice at a time."""
    rows, cols = 200, 16384
    w = si_hip.synth_matrix(Q6, seed=4242, rows=rows, cols=cols, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, Q6)
    base = si_hip.synth_normal(4243, cols)
    try:
        x = base.copy()
        x[100:140] = np.float32(3e30)            # slice 0
        x[4096 + 7] = np.float32(1e-9)           # slice 1: side elements
        x[4096 + 300:4096 + 303] = np.float32(-2e-10)
        x[8192:8192 + 256] = np.float32(1e-41)   # slice 2: a subnormal block
        x[12288 + 512:12288 + 768] = 0.0         # slice 3: a zero block
        _, y64, ab = O.matvec(Q6, w, rows, cols, x, threads=8)
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        assert_dot_close(y, y64, ab, what="special blocks")
        for k, v in [(50, np.inf), (4200, -np.inf), (9000, np.nan), (16383, np.inf)]:
            x = base.copy()
            x[k] = v
            y32, _, _ = O.matvec(Q6, w, rows, cols, x, threads=8)
            y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
            assert np.array_equal(_category(y), _category(y32)), f"x[{k}] = {v}"
    finally:
        W.free()


def test_sliced_and_split_launches_interleaved(hip_ctx):
    """Sliced launches share the workspace's tile counters and entries with
    the split launches of other shapes: each must find them reset, in any
    order and at any grid size."""
    cases = [(Q6, 2560, 17408), (Q4, 17408, 5120), (Q6, 16, 12288), (Q6, 151936 // 8, 5120),
             (Q6, 5120, 17408), (Q4, 1600, 17408), (Q6, 1000, 12800), (Q6, 2048, 32768)]
    mats = {}
    for t, rows, cols in cases:
        w = si_hip.synth_matrix(t, seed=rows + cols + t, rows=rows, cols=cols, threads=8)
        x = si_hip.synth_normal(rows ^ cols, cols)
        _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
        mats[(t, rows, cols)] = (hip_ctx.upload_quant_weight_private(w, t), x, y64, ab)
    try:
        for key in cases * 2:
            W, x, y64, ab = mats[key]
            t, rows, cols = key
            y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
            assert_dot_close(y, y64, ab, what=f"type {t} {rows}x{cols}")
    finally:
        for W, *_ in mats.values():
            W.free()


def test_sliced_down_in_fused_mlp(hip_ctx):
    """A fused MLP whose Q6_K down projection (17408 -> 2560) runs sliced:
    the output against the oracle's down projection of the device's own
    intermediate (bit-identical to the separate gate/up call's)."""
    inter, hidden = 17408, 2560
    g = si_hip.synth_matrix(Q4, seed=91, rows=inter, cols=hidden, threads=8)
    u = si_hip.synth_matrix(Q4, seed=92, rows=inter, cols=hidden, threads=8)
    d = si_hip.synth_matrix(Q6, seed=93, rows=hidden, cols=inter, threads=8)
    x = si_hip.synth_normal(94, hidden)
    G = hip_ctx.upload_quant_weight_private(g, Q4)
    U = hip_ctx.upload_quant_weight_private(u, Q4)
    D = hip_ctx.upload_quant_weight_private(d, Q6)
    try:
        h = hip_ctx.q4_k_fused_gate_up_weights(G, U, inter, hidden, x)
        y = hip_ctx.gguf_quant_fused_mlp_weights(G, U, D, inter, hidden, hidden, x)
        # the down projection of the device's own h, so only the down's error counts
        _, y64, ab = O.matvec(Q6, d, hidden, inter, h, threads=8)
        assert_dot_close(y, y64, ab, what="fused MLP down")
    finally:
        for m in (G, U, D):
            m.free()


def test_token_stage_combines_interleaved(hip_ctx):
    """Q4_K matmul-many of 3 to 16 vectors (one workgroup per stage and tile
    group, stage sums through the workspace's scratch) between K-sliced Q6_K
    and split Q4_K launches that share the tile counters: every call matches
    the oracle and repeats its own bits."""
    mats = {}
    for t, rows, cols in ((Q4, 17408, 5120), (Q4, 1040, 5120), (Q6, 2560, 17408),
                          (Q4, 1600, 17408)):
        w = si_hip.synth_matrix(t, seed=rows + cols, rows=rows, cols=cols, threads=8)
        mats[(t, rows, cols)] = (w, hip_ctx.upload_quant_weight_private(w, t))
    seq = [((Q4, 17408, 5120), 16), ((Q6, 2560, 17408), 1), ((Q4, 1040, 5120), 4),
           ((Q4, 1600, 17408), 1), ((Q4, 17408, 5120), 3), ((Q4, 1040, 5120), 11)]
    try:
        first = {}
        for rep in range(2):
            for key, batch in seq:
                t, rows, cols = key
                w, W = mats[key]
                X = si_hip.synth_normal(rows * batch + cols, batch * cols).reshape(batch, cols)
                log(f"interleaved: type {t} {rows}x{cols} batch {batch}, pass {rep}")
                if batch == 1:
                    outs = [hip_ctx.gguf_quant_matvec_weight(W, rows, cols, X[0])]
                else:
                    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
                if rep == 0:
                    for b in sorted({0, batch // 2, batch - 1}):
                        _, y64, ab = O.matvec(t, w, rows, cols, X[b], threads=8)
                        assert_dot_close(outs[b], y64, ab, what=f"{key} batch {batch} vector {b}")
                    first[(key, batch)] = [o.copy() for o in outs]
                else:
                    assert all(same_bits(a, b) for a, b in zip(outs, first[(key, batch)]))
    finally:
        for _, W in mats.values():
            W.free()


def test_sliced_launches_in_a_graph(hip_ctx):
    """K-sliced Q4_K and Q6_K matvecs and a split Q4_K matvec recorded in one
    HIP graph and replayed three times, with eager sliced and split launches
    on the same workspace between the replays: every replay equals the eager
    run bit for bit (the tile counters and entries are left clean by every
    launch; no memset is recorded)."""
    import ctypes as C
    lib = si_hip.lib()
    P = C.c_void_p
    shapes = [(Q4, 5120, 17408), (Q6, 2560, 17408), (Q4, 17408, 5120), (Q4, 2560, 34816)]
    mats, ins, outs = [], [], []
    for t, rows, cols in shapes:
        w = si_hip.synth_matrix(t, seed=rows + cols + 7 * t, rows=rows, cols=cols, threads=8)
        mats.append((w, hip_ctx.upload_quant_weight_private(w, t)))
        x = si_hip.synth_normal(rows * 3 + cols, cols)
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
        log("sliced graph: capture")
        hip_ctx.capture_begin()
        enqueue()
        graph = hip_ctx.capture_end()
        try:
            for rep in range(3):
                clear()
                # eager sliced and split launches on the same workspace
                for k in (1, 2):
                    (t, rows, cols), (_, W), (_, d_x) = shapes[k], mats[k], ins[k]
                    assert lib.si_hip_quant_matvec_device(h, W.handle, rows, cols, P(d_x),
                                                          P(d_e)) == 0
                hip_ctx.synchronize()
                log(f"sliced graph replay {rep}")
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


@pytest.mark.parametrize("seed", range(12))
def test_random_long_and_odd_rows(hip_ctx, seed):
    """Seeded random types, row counts (even and odd, partial tiles) and block
    counts (odd, long, past 128): one-vector matvecs that land on the
    K-sliced, row-pair, split, whole-tile and generic launches, every row
    within the oracle's bound and repeating its own bits."""
    rng = np.random.default_rng(9500 + seed)
    t = int(rng.choice([Q4, Q5, Q6]))
    cols = 256 * int(rng.choice([9, 21, 43, 48, 50, 64, 68, 108, 129, 136]))
    rows = int(rng.integers(1, 2000))
    log(f"random long/odd seed={seed}: type {t} {rows}x{cols}")
    w = si_hip.synth_matrix(t, seed=9600 + seed, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(9700 + seed, cols)
    W = hip_ctx.upload_quant_weight_private(w, t)
    try:
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
        assert_dot_close(y, y64, ab, what=f"type {t} {rows}x{cols}")
        assert same_bits(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y)
    finally:
        W.free()
