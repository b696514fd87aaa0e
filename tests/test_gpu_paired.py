"""GPU: Q6_K matvecs with an odd number of blocks per row.

A Q6_K block is 210 bytes, so with an odd block count nb consecutive rows
alternate between 4-byte aligned and 2 bytes off.  Such a matrix with an
even row count runs on the matrix cores as row pairs: the launch sees
rows / 2 rows of 2 nb blocks (rows 2 r and 2 r + 1 back to back, which
start aligned), x sits twice in the image area, and each block's sum goes
to its own row of the pair -- the stage holding blocks nb - 1 and nb hands
one sum to each.  Long pair rows over few tiles, and every pair row past 128
blocks (nb > 64), run K-sliced: a workgroup holds the images of its slice's
stretch of the doubled x, and the slice hand-off carries both sums of each
row.  An odd row count over 64K blocks or more runs its first rows - 1 rows
as pairs and the last row alone (one workgroup); smaller odd row counts run
the generic kernel.

Bar: rows within 2e-5 * sum|w*x| of the f64 dot, +-inf / NaN rows where
per-weight f32 products give them, the same bits on every call, and the
fused head's token equal to the oracle's under both tie rules.
"""
import sys

import numpy as np
import pytest

import oracle_lib as O
import si_hip
from test_gpu_parity import _category, assert_dot_close, same_bits

pytestmark = pytest.mark.gpu

Q6 = 14


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# (rows, cols): one block per row (the single stage straddles the pair);
# 9 blocks over a partial tile of pairs (17 pairs); the Gemma-class head
# width 5376 (21 blocks); the Llama-2-7B down projection (43 blocks, K-sliced
# pairs); a head of 32000 rows (a split launch of 1000 pair tiles); odd row
# counts (generic below 64K blocks: 41 rows, three rows of one block, one row;
# pairs, then the last row alone: 4097 rows of sliced pairs, a 32001-row
# head); pair rows past 128 blocks, which must slice (67, 65 and 129 blocks;
# 135 blocks: eight slices), and the same with an odd row count
SHAPES = [(2, 256), (34, 2304), (1000, 5376), (4096, 11008), (32000, 5376), (41, 2304),
          (3, 256), (4097, 11008), (32001, 5376), (1, 2304),
          (100, 17152), (2560, 16640), (2, 33024), (40, 34560), (1001, 17152), (501, 34560)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_odd_block_count_within_tolerance(hip_ctx, rows, cols):
    log(f"odd-nb q6_k {rows}x{cols}")
    w = si_hip.synth_matrix(Q6, seed=rows * 11 + cols, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(rows + 3 * cols, cols)
    _, y64, ab = O.matvec(Q6, w, rows, cols, x, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, Q6)
    try:
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        worst = assert_dot_close(y, y64, ab, what=f"{rows}x{cols}")
        log(f"  worst error / bound = {worst:.4f}")
        assert same_bits(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y)
    finally:
        W.free()


def test_odd_block_count_special_activations(hip_ctx):
    """Huge, side, subnormal and zero blocks, and single non-finite
    activations in the first block, the straddling stage's blocks (the last
    block of the even row, the first of the odd row) and the last block."""
    rows, cols = 64, 2304  # 9 blocks: the straddling stage holds block 8 and block 0
    w = si_hip.synth_matrix(Q6, seed=4400, rows=rows, cols=cols, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, Q6)
    base = si_hip.synth_normal(4401, cols)
    try:
        x = base.copy()
        x[100:140] = np.float32(3e30)
        x[300] = np.float32(1e-9)
        x[310:313] = np.float32(-2e-10)
        x[1024:1280] = np.float32(1e-41)
        x[2048:2304] = 0.0
        _, y64, ab = O.matvec(Q6, w, rows, cols, x, threads=8)
        assert_dot_close(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y64, ab,
                         what="special blocks")
        for k, v in [(5, np.inf), (2100, -np.inf), (2303, np.nan), (700, np.inf)]:
            x = base.copy()
            x[k] = v
            y32, _, _ = O.matvec(Q6, w, rows, cols, x, threads=8)
            y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
            assert np.array_equal(_category(y), _category(y32)), f"x[{k}] = {v}"
    finally:
        W.free()


def test_sliced_pairs_special_activations(hip_ctx):
    """Huge, side, subnormal and zero blocks across the slices of 67-block
    pair rows, including the straddling stage (blocks 66 and 67 of a pair
    row), then one infinite or NaN activation at a time."""
    rows, cols = 200, 17152
    w = si_hip.synth_matrix(Q6, seed=4600, rows=rows, cols=cols, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, Q6)
    base = si_hip.synth_normal(4601, cols)
    try:
        x = base.copy()
        x[100:140] = np.float32(3e30)
        x[4096 + 7] = np.float32(1e-9)
        x[4096 + 300:4096 + 303] = np.float32(-2e-10)
        x[8192:8192 + 256] = np.float32(1e-41)
        x[cols - 256:] = 0.0
        _, y64, ab = O.matvec(Q6, w, rows, cols, x, threads=8)
        assert_dot_close(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y64, ab,
                         what="special blocks")
        for k, v in [(5, np.inf), (cols - 1, -np.inf), (9000, np.nan), (256 * 33 + 3, np.inf)]:
            x = base.copy()
            x[k] = v
            y32, _, _ = O.matvec(Q6, w, rows, cols, x, threads=8)
            y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
            assert np.array_equal(_category(y), _category(y32)), f"x[{k}] = {v}"
    finally:
        W.free()


def test_odd_rows_split_special_activations(hip_ctx):
    """An odd row count split into sliced pairs and the last row alone: huge,
    side and zero blocks within the bound, then one infinite or NaN
    activation at a time, every row (the last one's own launch included) in
    the category that per-weight f32 products give."""
    rows, cols = 1001, 17152
    w = si_hip.synth_matrix(Q6, seed=4650, rows=rows, cols=cols, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, Q6)
    base = si_hip.synth_normal(4651, cols)
    try:
        x = base.copy()
        x[100:140] = np.float32(3e30)
        x[4096 + 7] = np.float32(1e-9)
        x[cols - 256:] = 0.0
        _, y64, ab = O.matvec(Q6, w, rows, cols, x, threads=8)
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        assert_dot_close(y, y64, ab, what="special blocks")
        for k, v in [(5, np.inf), (cols - 1, np.nan), (256 * 40 + 3, -np.inf)]:
            x = base.copy()
            x[k] = v
            y32, _, _ = O.matvec(Q6, w, rows, cols, x, threads=8)
            y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
            assert np.array_equal(_category(y), _category(y32)), f"x[{k}] = {v}"
    finally:
        W.free()


def test_sliced_pairs_in_a_graph(hip_ctx):
    """Sliced row pairs (32-float workspace entries), a plain sliced Q6_K
    launch (16-float entries) and an odd row count (sliced pairs, then the
    last row's generic launch) on one workspace, recorded in a HIP graph and
    replayed three times with eager launches between: every replay equals
    the eager run bit for bit (both leave the entries empty)."""
    import ctypes as C
    lib = si_hip.lib()
    P = C.c_void_p
    shapes = [(4096, 11008), (2560, 17408), (100, 17152), (1001, 17152)]
    mats, ins, outs = [], [], []
    for rows, cols in shapes:
        w = si_hip.synth_matrix(Q6, seed=rows + cols + 5, rows=rows, cols=cols, threads=8)
        mats.append((w, hip_ctx.upload_quant_weight_private(w, Q6)))
        x = si_hip.synth_normal(rows * 5 + cols, cols)
        d_x = hip_ctx.device_alloc(cols * 4)
        hip_ctx.to_device(d_x, x)
        ins.append((x, d_x))
        outs.append(hip_ctx.device_alloc(rows * 4))
    d_e = hip_ctx.device_alloc(4096 * 4)
    h = hip_ctx.handle

    def enqueue():
        for (rows, cols), (_, W), (_, d_x), d_y in zip(shapes, mats, ins, outs):
            rc = lib.si_hip_quant_matvec_device(h, W.handle, rows, cols, P(d_x), P(d_y))
            assert rc == 0, si_hip.last_error()

    def results():
        hip_ctx.synchronize()
        return [hip_ctx.from_device(d_y, rows) for (rows, _), d_y in zip(shapes, outs)]

    try:
        enqueue()
        ref = results()
        for (rows, cols), (w, _), (x, _), y in zip(shapes, mats, ins, ref):
            _, y64, ab = O.matvec(Q6, w, rows, cols, x, threads=8)
            assert_dot_close(y, y64, ab, what=f"eager {rows}x{cols}")
        hip_ctx.capture_begin()
        enqueue()
        graph = hip_ctx.capture_end()
        try:
            for rep in range(3):
                for (rows, _), d_y in zip(shapes, outs):
                    hip_ctx.to_device(d_y, np.full(rows, np.nan, np.float32))
                (rows, cols), (_, W), (_, d_x) = shapes[0], mats[0], ins[0]
                assert lib.si_hip_quant_matvec_device(h, W.handle, rows, cols, P(d_x), P(d_e)) == 0
                hip_ctx.synchronize()
                log(f"sliced pairs graph replay {rep}")
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


@pytest.mark.parametrize("rows,cols", [(20000, 2304), (4098, 5376)])
def test_odd_block_count_head_argmax(hip_ctx, rows, cols):
    """The output head with the argmax fused into the paired launch: the
    token is the oracle's argmax of the logits the call returns, under both
    tie rules, the logits repeat their bits and meet the bound (the plain
    matvec of the same head may run K-sliced, so it agrees within the bound);
    crafted ties across even and odd rows."""
    w = si_hip.synth_matrix(Q6, seed=rows + cols, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(rows - cols, cols)
    H = hip_ctx.upload_quant_weight_private(w, Q6)
    try:
        y = hip_ctx.gguf_quant_matvec_weight(H, rows, cols, x)
        _, y64, ab = O.matvec(Q6, w, rows, cols, x, threads=8)
        assert_dot_close(y, y64, ab, what="head logits")
        first = None
        for rule, pick in ((si_hip.ARGMAX_LAST_FINITE, O.argmax_last_finite),
                           (si_hip.ARGMAX_FIRST_GREATER, O.argmax_first_greater)):
            tok, logits = hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x, rule=rule)
            assert tok == pick(logits)
            assert_dot_close(logits, y64, ab, what="fused head logits")
            if first is None:
                first = logits
            assert same_bits(logits, first)
    finally:
        H.free()
    # ties: rows 7 (odd), 10 (even) and rows - 1 (odd) carry the same largest row
    nb = cols // 256
    blocks = np.asarray(w).reshape(rows, nb, 210).copy()
    big = bytearray(210)
    big[0:128] = b"\xff" * 128
    big[128:192] = b"\xff" * 64
    big[192:208] = bytes([127]) * 16
    big[208:210] = np.float16(1.0).tobytes()
    for r in (7, 10, rows - 1):
        blocks[r, :] = np.frombuffer(bytes(big), np.uint8)
    ones = np.ones(cols, np.float32)
    H = hip_ctx.upload_quant_weight_private(blocks.tobytes(), Q6)
    try:
        last, logits = hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, ones)
        first, _ = hip_ctx.gguf_quant_matvec_argmax_weight(
            H, rows, cols, ones, rule=si_hip.ARGMAX_FIRST_GREATER, want_logits=False)
        assert logits[7] == logits[10] == logits[rows - 1] == logits.max()
        assert (first, last) == (7, rows - 1)
    finally:
        H.free()


def test_odd_block_count_matmul_many(hip_ctx):
    """Several vectors over an odd-block matrix: one paired launch per
    vector, each within its bound."""
    rows, cols, batch = 1000, 5376, 3
    w = si_hip.synth_matrix(Q6, seed=4500, rows=rows, cols=cols, threads=8)
    X = si_hip.synth_normal(4501, batch * cols).reshape(batch, cols)
    W = hip_ctx.upload_quant_weight_private(w, Q6)
    try:
        outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
        for b in range(batch):
            _, y64, ab = O.matvec(Q6, w, rows, cols, X[b], threads=8)
            assert_dot_close(outs[b], y64, ab, what=f"vector {b}")
    finally:
        W.free()


@pytest.mark.parametrize("seed", range(8))
def test_random_odd_block_counts(hip_ctx, seed):
    """Seeded random Q6_K shapes with odd block counts and row counts of either
    parity up to 300K blocks: unsliced and sliced row pairs, the odd row
    count's pairs plus one-workgroup last row, and the generic kernel below
    64K blocks; every row within the oracle's bound and repeating its bits."""
    rng = np.random.default_rng(9800 + seed)
    nb = int(rng.choice([1, 9, 21, 43, 67, 135]))
    rows = int(rng.integers(1, min(8000, 300000 // nb) + 1))
    rows = rows | 1 if seed % 2 == 0 else max(2, rows & ~1)  # odd, then even row counts
    cols = 256 * nb
    log(f"random odd-nb q6_k seed={seed}: {rows}x{cols}")
    w = si_hip.synth_matrix(Q6, seed=9850 + seed, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(9870 + seed, cols)
    W = hip_ctx.upload_quant_weight_private(w, Q6)
    try:
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        _, y64, ab = O.matvec(Q6, w, rows, cols, x, threads=8)
        assert_dot_close(y, y64, ab, what=f"{rows}x{cols}")
        assert same_bits(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y)
    finally:
        W.free()
