"""GPU parity: the HIP path against the CPU oracle, through the C ABI.

Bars: dequantisation bit-exact with quant.rs; every
f32 dot within 2e-5 * sum|w*x| of the f64 value of the exact products;
greedy argmax identical.  Tests that restate the reference's own Metal tests
(src/metal.rs:7445-7602) keep their inputs and tolerances.
"""
import gc
import json
import struct
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle_lib as O
import si_hip

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
DOT_TOL = 2e-5          # relative to sum |w*x|
POLICIES = [si_hip.KERNEL_AUTO, si_hip.KERNEL_GENERIC]


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (a.view(np.uint32) == b.view(np.uint32))))


def assert_dot_close(y, y64, absdot, tol=DOT_TOL, what=""):
    err = np.abs(y.astype(np.float64) - y64)
    bound = tol * absdot + 1e-30
    worst = np.max(err / bound)
    assert worst <= 1.0, f"{what}: worst error {worst:.3f}x of {tol} * sum|w*x|"
    return worst


@pytest.fixture(params=POLICIES, ids=["auto", "generic"])
def ctx(request, hip_ctx):
    hip_ctx.set_kernel_policy(request.param)
    yield hip_ctx
    hip_ctx.set_kernel_policy(si_hip.KERNEL_AUTO)


# ---- dequantisation: bit-exact ------------------------------------------------
@pytest.mark.parametrize("t,name", [(12, "q4_k"), (13, "q5_k"), (14, "q6_k")])
def test_dequantize_fixtures_bit_exact(hip_ctx, t, name):
    log(f"dequant fixtures {name}")
    fx = json.loads((GOLDEN / f"blocks_{name}.json").read_text())
    data = bytes.fromhex(fx["bytes"])
    got = hip_ctx.dequantize(t, data, fx["n_blocks"] * 256)
    exp = np.array(fx["expected_bits"], dtype=np.uint32).view(np.float32)
    assert same_bits(got, exp)


def test_dequantize_reference_kats(hip_ctx):
    kats = json.loads((GOLDEN / "quant_kats.json").read_text())
    for k in kats["kats"]:
        got = hip_ctx.dequantize(k["ggml_type"], bytes.fromhex(k["bytes"]), k["elements"])
        assert np.array_equal(got, np.array(k["expected"], np.float32)), k["name"]
    for r in kats["rejections"]:
        with pytest.raises(si_hip.HipError):
            hip_ctx.dequantize(r["ggml_type"], bytes(r["byte_len"]), r["elements"])


@pytest.mark.parametrize("t", [12, 13, 14])
def test_dequantize_random_blocks_bit_exact(hip_ctx, t):
    log(f"dequant random type {t}")
    data = si_hip.synth_blocks(t, seed=900 + t, n_blocks=4096)
    got = hip_ctx.dequantize(t, data, 4096 * 256)
    assert same_bits(got, O.dequantize(t, data, 4096 * 256))
    # fully random bytes (NaN/inf d included)
    raw = np.random.default_rng(t).integers(0, 256, 1024 * si_hip.BLOCK_BYTES[t], dtype=np.uint8)
    assert same_bits(hip_ctx.dequantize(t, raw, 1024 * 256), O.dequantize(t, raw, 1024 * 256))


# ---- matvec ---------------------------------------------------------------------
# K from one block to past the tuned kernels' register-resident limit (32768)
# (odd block counts leave the matrix-core kernels a half-empty last stage)
SHAPES = [(1, 256), (7, 512), (64, 1024), (40, 2304), (300, 5120), (48, 5376), (1024, 5120),
          (33, 9216), (129, 17408), (17, 27648), (5, 33024)]


@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_matvec_within_tolerance(ctx, t, rows, cols):
    log(f"matvec t={t} {rows}x{cols}")
    w = si_hip.synth_matrix(t, seed=rows * 31 + cols + t, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(rows + 7 * t, cols)
    _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
    y = ctx.gguf_quant_matvec_bytes(t, w, rows, cols, x)
    assert_dot_close(y, y64, ab, what=f"type {t} {rows}x{cols}")
    weight = ctx.upload_quant_weight_private(w, t)
    y2 = ctx.gguf_quant_matvec_weight(weight, rows, cols, x)
    assert np.array_equal(y, y2)


@pytest.mark.parametrize("rows,cols", [(17408, 5120), (5120, 5120), (5120, 17408), (1024, 5120)])
def test_q4_k_baseline_shapes(hip_ctx, rows, cols):
    log(f"q4_k baseline shape {rows}x{cols}")
    w = si_hip.synth_matrix(12, seed=2024, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(5, cols)
    _, y64, ab = O.matvec(12, w, rows, cols, x, threads=8)
    weight = hip_ctx.upload_quant_weight_private(w, 12)
    y = hip_ctx.gguf_quant_matvec_weight(weight, rows, cols, x)
    worst = assert_dot_close(y, y64, ab, what=f"{rows}x{cols}")
    log(f"  worst error / bound = {worst:.4f}")


# the Q6_K output head (Qwen-style vocabulary) and MLP down projection
@pytest.mark.parametrize("rows,cols", [(5120, 17408), (151936, 5120)])
def test_q6_k_baseline_shapes(hip_ctx, rows, cols):
    log(f"q6_k baseline shape {rows}x{cols}")
    w = si_hip.synth_matrix(14, seed=2025, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(6, cols)
    _, y64, ab = O.matvec(14, w, rows, cols, x, threads=8)
    weight = hip_ctx.upload_quant_weight_private(w, 14)
    y = hip_ctx.gguf_quant_matvec_weight(weight, rows, cols, x)
    worst = assert_dot_close(y, y64, ab, what=f"{rows}x{cols}")
    log(f"  worst error / bound = {worst:.4f}")


def _category(v):
    v = np.asarray(v, np.float64)
    return np.where(np.isnan(v), 3, np.where(np.isposinf(v), 1, np.where(np.isneginf(v), 2, 0)))


# Q6_K rows of 48 blocks or more, where each wave converts its own pairs' x
# blocks: one tile, fewer pairs than waves, ragged tiles, a long grid
@pytest.mark.parametrize("rows,cols", [(16, 12288), (7, 16384), (300, 13312), (1040, 24576)])
def test_q6_k_long_rows(hip_ctx, rows, cols):
    log(f"q6_k long rows {rows}x{cols}")
    w = si_hip.synth_matrix(14, seed=rows + cols, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(rows + 11, cols)
    _, y64, ab = O.matvec(14, w, rows, cols, x, threads=8)
    weight = hip_ctx.upload_quant_weight_private(w, 14)
    y = hip_ctx.gguf_quant_matvec_weight(weight, rows, cols, x)
    assert_dot_close(y, y64, ab, what=f"{rows}x{cols}")
    weight.free()


def test_q6_k_long_rows_special_activations(hip_ctx):
    """The blocks a long row's waves convert themselves: huge (exact path),
    subnormal, zero and rounded blocks (a large element among tiny ones) within
    the bound, and one infinite or NaN activation giving +-inf / NaN rows
    exactly where per-weight f32 products do."""
    rows, cols = 80, 17408
    log("q6_k long rows, special activations")
    w = si_hip.synth_matrix(14, seed=1960, rows=rows, cols=cols, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, 14)
    base = si_hip.synth_normal(1961, cols)
    x = base.copy()
    x[600:620] = np.float32(3e30)
    x[621] = np.float32(-2.5e33)
    x[1024:1280] = np.float32(1e-41)
    x[1280:1536] = 0.0
    x[9000:9256] *= np.float32(1e-7)     # rounded: one element far above the rest
    x[9100] = np.float32(40.0)
    x[17000:17152] *= np.float32(1e-6)   # half a block tiny
    _, y64, ab = O.matvec(14, w, rows, cols, x, threads=8)
    y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
    assert_dot_close(y, y64, ab, what="huge/subnormal/rounded activations")
    for k, v in [(300, np.inf), (12000, -np.inf), (17407, np.nan)]:
        x = base.copy()
        x[k] = v
        y32, _, _ = O.matvec(14, w, rows, cols, x, threads=8)
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        assert np.array_equal(_category(y), _category(y32)), f"x[{k}] = {v}"
    W.free()


@pytest.mark.parametrize("policy", POLICIES)
def test_fused_gate_up_nonfinite_activations(hip_ctx, policy):
    """h = silu(gate.x) * (up.x) with an infinite or NaN activation: +-inf /
    NaN in the same rows as the per-weight f32 products and the reference's
    g / (1 + exp(-g)) * u (runtime.rs:4296-4298) give."""
    rows, cols = 48, 2304
    g = si_hip.synth_matrix(12, seed=31, rows=rows, cols=cols)
    u = si_hip.synth_matrix(12, seed=32, rows=rows, cols=cols)
    G = hip_ctx.upload_quant_weight_private(g, 12)
    U = hip_ctx.upload_quant_weight_private(u, 12)
    hip_ctx.set_kernel_policy(policy)
    try:
        for k, v in ((300, np.inf), (700, -np.inf), (1500, np.nan)):
            x = si_hip.synth_normal(33, cols).copy()
            x[k] = v
            h = hip_ctx.q4_k_fused_gate_up_weights(G, U, rows, cols, x)
            g32, _, _ = O.matvec(12, g, rows, cols, x)
            u32, _, _ = O.matvec(12, u, rows, cols, x)
            with np.errstate(all="ignore"):
                ref = (g32 / (np.float32(1) + np.exp(-g32)) * u32).astype(np.float32)
            assert np.array_equal(_category(h), _category(ref)), f"x[{k}] = {v}"
    finally:
        hip_ctx.set_kernel_policy(si_hip.KERNEL_AUTO)


@pytest.mark.parametrize("cols", [27648, 31744])
def test_nonfinite_activations_beyond_the_matrix_core_budget(hip_ctx, cols):
    """Q4_K with K of 27648 and 31744 (one tile: the launch is K-sliced, each
    workgroup holding a quarter of the row's images): an infinite activation
    gives +-inf rows by weight sign (NaN where a product is 0 * inf), as the
    reference's per-weight products do."""
    rows = 16
    w = si_hip.synth_matrix(12, seed=cols, rows=rows, cols=cols)
    W = hip_ctx.upload_quant_weight_private(w, 12)
    x = si_hip.synth_normal(cols + 1, cols).copy()
    x[300] = np.inf
    y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
    y32, _, _ = O.matvec(12, w, rows, cols, x)
    assert np.array_equal(_category(y), _category(y32))


@pytest.mark.parametrize("t", [12, 13, 14])
def test_matvec_nonfinite_and_huge_activations(ctx, t):
    """Blocks whose activations are not finite, or so large that a fixed-point
    form would overflow, or subnormal, must give what per-weight f32 products
    give: +-inf / NaN rows exactly where the reference has them, and finite rows
    within the usual bound."""
    rows, cols = 48, 2304
    log(f"non-finite activations t={t}")
    w = si_hip.synth_matrix(t, seed=1900 + t, rows=rows, cols=cols)
    W = ctx.upload_quant_weight_private(w, t)
    base = si_hip.synth_normal(1901, cols)
    # huge (>= 2^100) values in one block, subnormal and zero blocks elsewhere
    x = base.copy()
    x[600:620] = np.float32(3e30)
    x[621] = np.float32(-2.5e33)
    x[1024:1280] = np.float32(1e-41)
    x[1280:1536] = 0.0
    _, y64, ab = O.matvec(t, w, rows, cols, x)
    y = ctx.gguf_quant_matvec_weight(W, rows, cols, x)
    assert_dot_close(y, y64, ab, what="huge/subnormal activations")
    # one infinite activation: the sign of w[r, k] decides +inf / -inf, w == 0 gives NaN
    for k, v in [(300, np.inf), (1800, -np.inf), (5, np.nan)]:
        x = base.copy()
        x[k] = v
        y32, _, _ = O.matvec(t, w, rows, cols, x)
        y = ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        assert np.array_equal(_category(y), _category(y32)), f"x[{k}] = {v}"


def test_matvec_outlier_activations_on_zero_weights(ctx):
    """Massive activations whose Q6_K weights are exactly zero (q = 32): the
    dot is then carried by the ordinary activations alone, which must keep
    full precision next to the outlier (quant.rs:155-169 decoding)."""
    rows, cols = 64, 2048
    w = bytearray(si_hip.synth_matrix(14, seed=1950, rows=rows, cols=cols))
    nb = cols // 256
    outliers = [3, 300, 777, 1100, 2047]
    for r in range(rows):
        for k in outliers:
            blk, e = divmod(k, 256)
            h, rem = divmod(e, 128)
            t, l = divmod(rem, 32)
            base = (r * nb + blk) * 210
            qi = base + 64 * h + l + 32 * (t & 1)
            w[qi] &= 0xF0 if (t >> 1) == 0 else 0x0F           # nibble 0
            hi = base + 128 + 32 * h + l
            w[hi] = (w[hi] & ~(3 << (2 * t)) & 0xFF) | (2 << (2 * t))  # high bits 2 -> q = 32
    w = bytes(w)
    dq = O.dequantize(14, w, rows * cols).reshape(rows, cols)
    assert np.all(dq[:, outliers] == 0.0)
    x = si_hip.synth_normal(1951, cols)
    x[outliers] = np.float32(1e6)
    _, y64, ab = O.matvec(14, w, rows, cols, x)
    W = ctx.upload_quant_weight_private(w, 14)
    y = ctx.gguf_quant_matvec_weight(W, rows, cols, x)
    assert_dot_close(y, y64, ab, what="outliers on zero weights")


def test_split_tiles_across_grid_sizes(hip_ctx):
    """Launches with large, then small grids, with and without split tiles:
    tiles whose partials span several workgroups are combined through per-tile
    counters and entries that every launch must find reset, whatever the
    previous launch's grid was."""
    cases = [(12, 17408, 5120), (14, 160, 17408), (12, 1600, 17408), (14, 48, 17408),
             (12, 160, 17408), (14, 300, 5120), (12, 48, 17408), (12, 1024, 5120),
             (14, 5120, 17408), (12, 40, 2304), (14, 16, 512)]
    for t, rows, cols in cases * 2:
        w = si_hip.synth_matrix(t, seed=rows + cols + t, rows=rows, cols=cols, threads=8)
        x = si_hip.synth_normal(rows ^ cols, cols)
        _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
        W = hip_ctx.upload_quant_weight_private(w, t)
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        assert_dot_close(y, y64, ab, what=f"type {t} {rows}x{cols}")


def test_matvec_cancellation_heavy_blocks(ctx):
    # blocks where d*sc*q and dmin*m nearly cancel: all nibbles equal, m chosen
    # so that w is small against its two terms
    rows, cols = 16, 2048
    rng = np.random.default_rng(11)
    blocks = []
    for r in range(rows * cols // 256):
        b = bytearray(144)
        b[0:2] = struct.pack("<e", 0.01 + 0.001 * (r % 5))
        b[2:4] = struct.pack("<e", 0.01 + 0.001 * (r % 5))
        sc = [int(v) for v in rng.integers(20, 64, 8)]
        q = int(rng.integers(1, 16))
        mn = [min(63, s * q // 4) for s in sc]
        import numpy_ref
        b[4:16] = numpy_ref.encode_k4_scales(sc, mn)
        b[16:] = bytes([(q | (q << 4))] * 128)
        # sprinkle different nibbles so rows are not all-constant
        for i in rng.integers(0, 128, 12):
            b[16 + int(i)] = int(rng.integers(0, 256))
        blocks.append(bytes(b))
    w = b"".join(blocks)
    x = si_hip.synth_normal(99, cols)
    _, y64, ab = O.matvec(12, w, rows, cols, x)
    y = ctx.q4_k_matvec(w, rows, cols, x)
    assert_dot_close(y, y64, ab, what="cancellation")


# restatement of metal.rs:7445-7494 (q4_k_matvec_kernel_matches_cpu_reference)
def test_reference_q4_k_matvec_test(ctx):
    rows, cols = 2, 512
    w = bytearray(rows * 2 * 144)
    for row in range(rows):
        for bi in range(2):
            s = (row * 2 + bi) * 144
            w[s:s + 2] = struct.pack("<H", 0x3C00)
            for i in range(12):
                w[s + 4 + i] = (i * 13 + 7) & 0xFF
            for i in range(128):
                w[s + 16 + i] = 0x10 if (i + row + bi) % 3 == 0 else 0x21
    x = np.array([((i % 11) - 5.0) / 3.0 for i in range(cols)], np.float32)
    expected, _, _ = O.matvec(12, bytes(w), rows, cols, x)
    got = ctx.q4_k_matvec(bytes(w), rows, cols, x)
    assert np.all(np.abs(got - expected) < 1e-4)


# restatement of metal.rs:7565-7602 (q5_and_q6_k_matvec_kernels_match_cpu_reference)
def test_reference_q5_q6_matvec_test(ctx):
    x = np.array([((i % 13) - 6.0) / 5.0 for i in range(256)], np.float32)
    q5 = bytearray(176)
    q5[0:2] = struct.pack("<H", 0x3C00)
    q5[4:16] = bytes([1] * 12)
    q5[16:48] = bytes([0xFF] * 32)
    q5[48:] = bytes([0x10] * 128)
    e5, _, _ = O.matvec(13, bytes(q5), 1, 256, x)
    assert abs(ctx.q5_k_matvec(bytes(q5), 1, 256, x)[0] - e5[0]) < 1e-4
    q6 = bytearray(210)
    q6[208:210] = struct.pack("<H", 0x3C00)
    q6[:128] = bytes([0x21] * 128)
    q6[128:192] = bytes([0xE4] * 64)
    q6[192:208] = bytes([1] * 16)
    e6, _, _ = O.matvec(14, bytes(q6), 1, 256, x)
    assert abs(ctx.q6_k_matvec(bytes(q6), 1, 256, x)[0] - e6[0]) < 1e-4


# ---- fused SwiGLU -----------------------------------------------------------------
def silu64(g):
    return g / (1.0 + np.exp(-g))


def gate_up_bound(g64, ag, u64, au):
    sig = 1.0 / (1.0 + np.exp(-g64))
    dsilu = np.abs(sig * (1.0 + g64 * (1.0 - sig)))
    return DOT_TOL * (dsilu * ag * np.abs(u64) + np.abs(silu64(g64)) * au) \
        + 4e-7 * np.abs(silu64(g64) * u64) + 1e-30


# restatement of metal.rs:7498-7540
def test_reference_fused_gate_up_test(ctx):
    rows, cols = 2, 256
    gate = bytearray(rows * 144)
    up = bytearray(rows * 144)
    for row in range(rows):
        s = row * 144
        gate[s:s + 2] = struct.pack("<H", 0x3C00)
        up[s:s + 2] = struct.pack("<H", 0x3800)
        gate[s + 4:s + 16] = bytes([7] * 12)
        up[s + 4:s + 16] = bytes([11] * 12)
        gate[s + 16:s + 144] = bytes([0x21] * 128)
        up[s + 16:s + 144] = bytes([0x12] * 128)
    x = np.array([((i % 17) - 8.0) / 5.0 for i in range(cols)], np.float32)
    g, _, _ = O.matvec(12, bytes(gate), rows, cols, x)
    u, _, _ = O.matvec(12, bytes(up), rows, cols, x)
    expected = np.array([O.silu(float(a)) * b for a, b in zip(g, u)], np.float32)
    got = ctx.q4_k_fused_gate_up(bytes(gate), bytes(up), rows, cols, x)
    assert np.all(np.abs(got - expected) < 1e-4)


@pytest.mark.parametrize("rows,cols", [(64, 1024), (1000, 5120), (160, 17408), (17408, 5120)])
def test_fused_gate_up_within_tolerance(ctx, rows, cols):
    log(f"gate/up {rows}x{cols}")
    gw = si_hip.synth_matrix(12, seed=501, rows=rows, cols=cols, threads=8)
    uw = si_hip.synth_matrix(12, seed=502, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(503, cols, scale=0.1)
    _, g64, ag = O.matvec(12, gw, rows, cols, x, threads=8)
    _, u64, au = O.matvec(12, uw, rows, cols, x, threads=8)
    g = ctx.upload_quant_weight_private(gw, 12)
    u = ctx.upload_quant_weight_private(uw, 12)
    h = ctx.q4_k_fused_gate_up_weights(g, u, rows, cols, x)
    ref = silu64(g64) * u64
    err = np.abs(h.astype(np.float64) - ref)
    assert np.all(err <= gate_up_bound(g64, ag, u64, au))


def test_fused_mlp_q6_down(ctx):
    gate_rows, cols, down_rows = 2048, 1024, 512
    log("fused mlp")
    gw = si_hip.synth_matrix(12, seed=601, rows=gate_rows, cols=cols, threads=8)
    uw = si_hip.synth_matrix(12, seed=602, rows=gate_rows, cols=cols, threads=8)
    dw = si_hip.synth_matrix(14, seed=603, rows=down_rows, cols=gate_rows, threads=8)
    x = si_hip.synth_normal(604, cols, scale=0.1)
    _, g64, ag = O.matvec(12, gw, gate_rows, cols, x, threads=8)
    _, u64, au = O.matvec(12, uw, gate_rows, cols, x, threads=8)
    h64 = silu64(g64) * u64
    hb = gate_up_bound(g64, ag, u64, au)
    wd = O.dequantize(14, dw, down_rows * gate_rows).reshape(down_rows, gate_rows).astype(np.float64)
    y64 = wd @ h64
    bound = DOT_TOL * (np.abs(wd) @ np.abs(h64)) + np.abs(wd) @ hb + 1e-30
    G = ctx.upload_quant_weight_private(gw, 12)
    U = ctx.upload_quant_weight_private(uw, 12)
    D = ctx.upload_quant_weight_private(dw, 14)
    y = ctx.gguf_quant_fused_mlp_weights(G, U, D, gate_rows, cols, down_rows, x)
    assert np.all(np.abs(y - y64) <= bound)


# ---- embedding ----------------------------------------------------------------------
# restatement of metal.rs:7544-7561 (bit-exact here: it is a dequantisation)
def test_reference_embedding_row_test(ctx):
    row = bytearray(144)
    row[0:2] = struct.pack("<H", 0x3C00)
    row[4:16] = bytes([7, 19, 31, 43, 55, 67, 79, 91, 103, 115, 127, 139])
    row[16:] = bytes([0x21] * 128)
    got = ctx.q4_k_embedding_row(bytes(row), 256)
    assert same_bits(got, O.dequantize(12, bytes(row), 256))


def test_embedding_tokens_bit_exact(hip_ctx):
    vocab, cols = 4099, 5120
    table = si_hip.synth_matrix(12, seed=700, rows=vocab, cols=cols, threads=8)
    T = hip_ctx.upload_quant_weight_private(table, 12)
    ids = si_hip.synth_token_ids(701, 64, vocab)
    ids[0], ids[1] = 0, vocab - 1
    got = hip_ctx.q4_k_embedding_tokens(T, (cols, vocab), ids)
    rb = cols // 256 * 144
    for i, t in enumerate(ids):
        exp = O.dequantize(12, table[t * rb:(t + 1) * rb], cols)
        assert same_bits(got[i], exp)
    one = hip_ctx.q4_k_embedding_tensor(T, (cols, vocab), int(ids[5]))
    assert same_bits(one, got[5])
    with pytest.raises(si_hip.HipError) as e:
        hip_ctx.q4_k_embedding_tensor(T, (cols, vocab), vocab)
    assert e.value.status == -7


# ---- multi-token verify --------------------------------------------------------------
@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("batch", [1, 2, 4, 8, 16])
def test_matmul_many(ctx, t, batch):
    rows, cols = 512, 5120
    log(f"matmul_many t={t} batch={batch}")
    w = si_hip.synth_matrix(t, seed=800 + t, rows=rows, cols=cols, threads=8)
    X = si_hip.synth_normal(801, batch * cols).reshape(batch, cols)
    W = ctx.upload_quant_weight_private(w, t)
    if batch <= 8:
        outs = ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    else:
        outs = ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(batch):
        _, y64, ab = O.matvec(t, w, rows, cols, X[b], threads=8)
        assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")


@pytest.mark.parametrize("rows,cols,batch", [(100, 2304, 3), (16, 256, 2), (1040, 5120, 4),
                                             (33, 1280, 7), (48, 9216, 2)])
def test_matmul_many_ragged_shapes(hip_ctx, rows, cols, batch):
    """Partial tiles, block counts that leave a short last stage, passes with
    fewer than four vectors, and a K whose images do not fit the LDS."""
    log(f"matmul_many ragged {rows}x{cols} batch={batch}")
    w = si_hip.synth_matrix(12, seed=rows * 7 + cols, rows=rows, cols=cols)
    X = si_hip.synth_normal(rows + batch, batch * cols).reshape(batch, cols)
    W = hip_ctx.upload_quant_weight_private(w, 12)
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(batch):
        _, y64, ab = O.matvec(12, w, rows, cols, X[b])
        assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")


def test_matmul_many_nonfinite_and_outlier_vectors(hip_ctx):
    """Blocks that must take the exact path in some vectors of a pass and
    not in others: huge, subnormal, outlier and non-finite activations."""
    rows, cols, batch = 48, 2304, 4
    w = si_hip.synth_matrix(12, seed=4242, rows=rows, cols=cols)
    W = hip_ctx.upload_quant_weight_private(w, 12)
    X = si_hip.synth_normal(4243, batch * cols).reshape(batch, cols).copy()
    X[1, 600:620] = np.float32(3e30)
    X[1, 1024:1280] = np.float32(1e-41)
    X[2, 300] = np.float32(1e6)
    X[2, 2000] = np.float32(-1e6)
    X[3, 700] = np.inf
    X[3, 1500] = np.nan
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(3):
        _, y64, ab = O.matvec(12, w, rows, cols, X[b])
        assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")
    y32, _, _ = O.matvec(12, w, rows, cols, X[3])
    assert np.array_equal(_category(outs[3]), _category(y32))


@pytest.mark.parametrize("rows,cols,batch", [(100, 2304, 3), (1040, 5120, 8), (33, 1280, 7),
                                             (300, 17408, 5), (5120, 5120, 16)])
def test_q5_k_matmul_many_vectors_in_rows(hip_ctx, rows, cols, batch):
    """Q5_K candidates in the matrix-core rows (the qh bit as the weights'
    fifth bit): partial tiles, a short last stage, K slices, a long K and
    sixteen vectors in one pass; repeat calls bit-identical."""
    log(f"q5_k matmul_many {rows}x{cols} batch={batch}")
    w = si_hip.synth_matrix(13, seed=rows * 11 + cols + batch, rows=rows, cols=cols, threads=8)
    X = si_hip.synth_normal(rows + 5 * batch, batch * cols).reshape(batch, cols)
    W = hip_ctx.upload_quant_weight_private(w, 13)
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    again = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(batch):
        _, y64, ab = O.matvec(13, w, rows, cols, X[b], threads=8)
        assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")
        assert np.array_equal(outs[b], again[b])


def test_q5_k_matmul_many_nonfinite_side_and_rounded(hip_ctx):
    """Eight Q5_K candidates: listed side elements, rounded blocks, huge,
    subnormal and zero blocks, and non-finite activations in some vectors
    only."""
    rows, cols, batch = 300, 5120, 8
    w = si_hip.synth_matrix(13, seed=4260, rows=rows, cols=cols, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, 13)
    X = si_hip.synth_normal(4261, batch * cols).reshape(batch, cols).copy()
    X[0, 256:259] = np.float32(3e-9)
    X[1, 512:540] = np.float32(2e-9)
    X[2, 1024:1280] = np.float32(1e-41)
    X[2, 2048:2304] = 0.0
    X[3, 600:620] = np.float32(3e30)
    X[4, 300] = np.float32(1e6)
    X[5] = 0.0
    X[6, 700] = np.inf
    X[7, 1500] = np.nan
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(6):
        _, y64, ab = O.matvec(13, w, rows, cols, X[b], threads=8)
        assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")
    assert not np.any(outs[5])
    for b in (6, 7):
        y32, _, _ = O.matvec(13, w, rows, cols, X[b], threads=8)
        assert np.array_equal(_category(outs[b]), _category(y32)), f"candidate {b}"


def test_matmul_many_baseline_shape(hip_ctx):
    """M = 6 candidates on the 17408 x 5120 Q4_K matrix: one pass over the
    weights for four vectors and one for two; each candidate matches its own
    reference and the batch is deterministic."""
    rows, cols, batch = 17408, 5120, 6
    w = si_hip.synth_matrix(12, seed=2026, rows=rows, cols=cols, threads=8)
    X = si_hip.synth_normal(2027, batch * cols).reshape(batch, cols)
    W = hip_ctx.upload_quant_weight_private(w, 12)
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    again = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(batch):
        _, y64, ab = O.matvec(12, w, rows, cols, X[b], threads=8)
        assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")
        assert np.array_equal(outs[b], again[b])


@pytest.mark.parametrize("rows,cols,batch", [(100, 2560, 3), (33, 512, 2), (1040, 5120, 7),
                                             (512, 5120, 16), (300, 17408, 2), (48, 2304, 3)])
def test_q6_k_matmul_many_shapes(hip_ctx, rows, cols, batch):
    """Q6_K candidates four, three or two per pass over the weights: partial
    tiles, a short K, the down projection's K (whose images do not fit two
    vectors: one per pass) and an odd block count (the generic kernel)."""
    log(f"q6_k matmul_many {rows}x{cols} batch={batch}")
    w = si_hip.synth_matrix(14, seed=rows * 3 + cols, rows=rows, cols=cols)
    X = si_hip.synth_normal(rows + 2 * batch, batch * cols).reshape(batch, cols)
    W = hip_ctx.upload_quant_weight_private(w, 14)
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    again = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(batch):
        _, y64, ab = O.matvec(14, w, rows, cols, X[b])
        assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")
        assert np.array_equal(outs[b], again[b])


def test_q6_k_matmul_many_nonfinite_and_outlier_vectors(hip_ctx):
    """Q6_K blocks on the exact path in some vectors of a pass and not in
    others."""
    rows, cols, batch = 48, 2560, 4
    w = si_hip.synth_matrix(14, seed=4244, rows=rows, cols=cols)
    W = hip_ctx.upload_quant_weight_private(w, 14)
    X = si_hip.synth_normal(4245, batch * cols).reshape(batch, cols).copy()
    X[0, 600:620] = np.float32(3e30)
    X[1, 1024:1280] = np.float32(1e-41)
    X[1, 300] = np.float32(1e6)
    X[2, 2000] = np.float32(-1e6)
    X[3, 700] = np.inf
    X[3, 1500] = np.nan
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(3):
        _, y64, ab = O.matvec(14, w, rows, cols, X[b])
        assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")
    y32, _, _ = O.matvec(14, w, rows, cols, X[3])
    assert np.array_equal(_category(outs[3]), _category(y32))


def test_q6_k_matmul_many_head_shape(hip_ctx):
    """Four candidates through the 151936 x 5120 Q6_K output head in one pass:
    each within the bound of the oracle."""
    rows, cols, batch = 151936, 5120, 4
    w = si_hip.synth_matrix(14, seed=2025, rows=rows, cols=cols, threads=8)
    X = si_hip.synth_normal(2030, batch * cols).reshape(batch, cols)
    W = hip_ctx.upload_quant_weight_private(w, 14)
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(batch):
        _, y64, ab = O.matvec(14, w, rows, cols, X[b], threads=8)
        worst = assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")
        log(f"  candidate {b}: worst error / bound = {worst:.4f}")


# Q6_K candidates up to eight per pass (the vectors in the matrix-core rows,
# K slices of four blocks summed by the reduce kernel): ragged tiles, fewer
# vectors than eight, two passes, the down projection's K and the head.
@pytest.mark.parametrize("rows,cols,batch", [(33, 2560, 3), (1000, 5120, 5), (100, 1024, 6),
                                             (4096, 4096, 16), (5120, 17408, 8),
                                             (1040, 2048, 11), (17, 512, 4), (40, 1536, 16),
                                             (2000, 5120, 13)])
def test_q6_k_matmul_many_eight_per_pass(hip_ctx, rows, cols, batch):
    log(f"q6_k matmul_many {rows}x{cols} batch={batch}")
    w = si_hip.synth_matrix(14, seed=rows * 5 + cols + batch, rows=rows, cols=cols, threads=8)
    X = si_hip.synth_normal(rows + 3 * batch, batch * cols).reshape(batch, cols)
    W = hip_ctx.upload_quant_weight_private(w, 14)
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    again = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(batch):
        _, y64, ab = O.matvec(14, w, rows, cols, X[b], threads=8)
        assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")
        assert np.array_equal(outs[b], again[b])


def test_q6_k_matmul_many_eight_side_rounded_and_exact_blocks(hip_ctx):
    """Eight Q6_K candidates in one pass whose blocks differ: listed side
    elements (a few tiny activations beside large ones), rounded blocks (more
    than eight), subnormal and zero blocks, blocks on the exact path (huge,
    infinite, NaN) in some vectors only, and a vector of zeros."""
    rows, cols, batch = 300, 5120, 8
    w = si_hip.synth_matrix(14, seed=4250, rows=rows, cols=cols, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, 14)
    X = si_hip.synth_normal(4251, batch * cols).reshape(batch, cols).copy()
    X[0, 256:259] = np.float32(3e-9)               # listed side elements
    X[0, 1000] = np.float32(-1e-12)
    X[1, 512:540] = np.float32(2e-9)               # a rounded block
    X[1, 4096:4352:3] = np.float32(-5e-10)         # another, spread out
    X[2, 1024:1280] = np.float32(1e-41)            # subnormal block
    X[2, 2048:2304] = 0.0                          # zero block
    X[3, 600:620] = np.float32(3e30)               # huge: exact path
    X[4] = 0.0
    X[5, 300] = np.float32(1e6)
    X[5, 301:309] = np.float32(1e-4)               # side elements of a large block
    X[6, 700] = np.inf
    X[7, 1500] = np.nan
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    again = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(6):
        _, y64, ab = O.matvec(14, w, rows, cols, X[b], threads=8)
        assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")
        assert np.array_equal(outs[b], again[b])
    assert not np.any(outs[4])
    for b in (6, 7):
        y32, _, _ = O.matvec(14, w, rows, cols, X[b], threads=8)
        assert np.array_equal(_category(outs[b]), _category(y32)), f"candidate {b}"


@pytest.mark.parametrize("batch", [8, 16])
def test_q6_k_matmul_many_head_eight(hip_ctx, batch):
    """Eight and sixteen candidates through the 151936 x 5120 Q6_K output
    head in one pass over its 638 MB: each within the bound of the oracle."""
    rows, cols = 151936, 5120
    w = si_hip.synth_matrix(14, seed=2026, rows=rows, cols=cols, threads=8)
    X = si_hip.synth_normal(2031, batch * cols).reshape(batch, cols)
    W = hip_ctx.upload_quant_weight_private(w, 14)
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(batch):
        _, y64, ab = O.matvec(14, w, rows, cols, X[b], threads=8)
        worst = assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")
        log(f"  candidate {b}: worst error / bound = {worst:.4f}")


@pytest.mark.parametrize("types,rows,cols", [
    ((12, 12, 12), (6144, 1024, 1024), 5120),   # one launch (two-block stages)
    ((12, 12), (8192, 8192), 5120),             # one launch (four-block stages)
    ((13, 13), (304, 200), 5376),               # Q5_K, one launch, an odd block count
    ((12, 12, 12), (16, 48, 33), 2304),         # one launch, ragged last matrix
    ((12,) * 8, (64,) * 7 + (100,), 1024),      # the largest group of one launch
    ((12, 12), (100, 64), 1024),                # first rows not whole tiles: one launch each
    ((12, 14, 13), (64, 32, 48), 2560),         # mixed types: one launch each
    ((13, 13, 13), (1024, 512, 300), 5120),     # Q5_K, one launch
    ((14, 14), (1024, 160), 17408),             # Q6_K, one launch (long K: L2 touch)
    ((14,) * 4, (64, 64, 64, 40), 2560),        # Q6_K, one launch
    ((14, 14), (48, 40), 2304),                 # Q6_K with an odd block count: one launch each
])
def test_grouped_matvec(hip_ctx, types, rows, cols):
    """Several matvecs over one input (gguf_quant_matvec_many_weights), as one
    matrix-core launch where the group allows it: every output within the
    bound of the oracle, the device-resident form bit-identical to the host
    form, and repeat calls deterministic."""
    log(f"grouped matvec types={types} rows={rows} cols={cols}")
    hosts = [si_hip.synth_matrix(t, seed=70 + i, rows=r, cols=cols)
             for i, (t, r) in enumerate(zip(types, rows))]
    ws = [hip_ctx.upload_quant_weight_private(w, t) for w, t in zip(hosts, types)]
    x = si_hip.synth_normal(71, cols)
    outs = hip_ctx.gguf_quant_matvec_many_weights(ws, rows, cols, x)
    for i, (t, r) in enumerate(zip(types, rows)):
        _, y64, ab = O.matvec(t, hosts[i], r, cols, x)
        assert_dot_close(outs[i], y64, ab, what=f"matrix {i}")
    total = sum(rows)
    d_x, d_y = hip_ctx.device_alloc(cols * 4), hip_ctx.device_alloc(total * 4)
    hip_ctx.to_device(d_x, x)
    for _ in range(2):
        hip_ctx.quant_matvec_many_device(ws, rows, cols, d_x, d_y)
        hip_ctx.synchronize()
        y = hip_ctx.from_device(d_y, (total,))
        assert np.array_equal(y, np.concatenate(outs))
    hip_ctx.device_free(d_x)
    hip_ctx.device_free(d_y)


@pytest.mark.parametrize("seed", range(6))
def test_random_shapes_batches_and_groups(hip_ctx, seed):
    """Seeded random types, shapes (partial tiles, short and long K, odd block
    counts), batches 1-16 and groups of 2-9 matrices: every output within the
    bound of the oracle.  Covers the choice between the one-vector, several-
    vector, vectors-in-rows, grouped and generic launches together."""
    rng = np.random.default_rng(9000 + seed)
    t = int(rng.choice([12, 13, 14]))
    cols = 256 * int(rng.choice([1, 2, 3, 9, 20, 36, 68]))
    rows = int(rng.integers(1, 700))
    batch = int(rng.integers(1, 17))
    log(f"random seed={seed}: type {t} {rows}x{cols} batch {batch}")
    w = si_hip.synth_matrix(t, seed=9100 + seed, rows=rows, cols=cols)
    X = si_hip.synth_normal(9200 + seed, batch * cols).reshape(batch, cols)
    W = hip_ctx.upload_quant_weight_private(w, t)
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(batch):
        _, y64, ab = O.matvec(t, w, rows, cols, X[b])
        assert_dot_close(outs[b], y64, ab, what=f"candidate {b}")
    n = int(rng.integers(2, 10))
    g_rows = [16 * int(rng.integers(1, 40)) for _ in range(n - 1)] + [int(rng.integers(1, 300))]
    g_types = [t] * n if rng.random() < 0.7 else [int(rng.choice([12, 13, 14])) for _ in range(n)]
    hosts = [si_hip.synth_matrix(tt, seed=9300 + 10 * seed + i, rows=r, cols=cols)
             for i, (tt, r) in enumerate(zip(g_types, g_rows))]
    ws = [hip_ctx.upload_quant_weight_private(hb, tt) for hb, tt in zip(hosts, g_types)]
    youts = hip_ctx.gguf_quant_matvec_many_weights(ws, g_rows, cols, X[0])
    for i, (tt, r) in enumerate(zip(g_types, g_rows)):
        _, y64, ab = O.matvec(tt, hosts[i], r, cols, X[0])
        assert_dot_close(youts[i], y64, ab, what=f"group matrix {i}")


def test_matmul_many_bytes_matches_weight(hip_ctx):
    rows, cols, batch = 96, 1024, 3
    w = si_hip.synth_matrix(13, seed=9, rows=rows, cols=cols)
    X = si_hip.synth_normal(10, batch * cols)
    a = hip_ctx.gguf_quant_matmul_many_bytes(13, w, rows, cols, batch, X)
    W = hip_ctx.upload_quant_weight_private(w, 13)
    b = hip_ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for i in range(batch):
        assert np.array_equal(a[i], b[i])


# ---- output head + argmax -----------------------------------------------------------
@pytest.mark.parametrize("t", [12, 14])
def test_head_argmax_matches_oracle(ctx, t):
    rows, cols = 20011, 5120
    log(f"head argmax t={t}")
    w = si_hip.synth_matrix(t, seed=1100 + t, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(1101, cols)
    y32, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
    H = ctx.upload_quant_weight_private(w, t)
    tok, logits = ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x)
    assert_dot_close(logits, y64, ab, what="head logits")
    order = np.argsort(y64)
    top, second = order[-1], order[-2]
    margin = y64[top] - y64[second]
    bound = DOT_TOL * (ab[top] + ab[second])
    log(f"  top-2 margin {margin:.6g} vs error bound {bound:.3g}")
    assert margin > bound
    assert tok == top == O.argmax_last_finite(y32) == O.argmax_last_finite(logits)
    tok2, _ = ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x, rule=si_hip.ARGMAX_FIRST_GREATER,
                                                  want_logits=False)
    assert tok2 == tok


def test_head_argmax_tie_rules(hip_ctx):
    # identical rows -> identical logits -> ties decided by the rule
    rows, cols = 4096 + 5, 256
    base = si_hip.synth_matrix(12, seed=1200, rows=rows, cols=cols)
    blocks = base.reshape(rows, 144).copy()
    # row 17: d = 1, dmin = 0, every scale and nibble at its maximum, so with
    # x = 1 its logit (63*15*256) dominates every random row (d ~ 0.02)
    blocks[17, 0:2] = np.frombuffer(struct.pack("<H", 0x3C00), np.uint8)
    blocks[17, 2:4] = 0
    blocks[17, 4:] = 0xFF
    blocks[1000] = blocks[17]
    blocks[3000] = blocks[17]
    x = np.ones(cols, np.float32)
    H = hip_ctx.upload_quant_weight_private(blocks.tobytes(), 12)
    _, logits = hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x)
    assert logits[17] == logits[1000] == logits[3000] == logits.max()
    last, _ = hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x, rule=si_hip.ARGMAX_LAST_FINITE)
    first, _ = hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x, rule=si_hip.ARGMAX_FIRST_GREATER)
    assert (first, last) == (17, 3000)
    assert last == O.argmax_last_finite(logits)
    assert first == O.argmax_first_greater(logits)


def test_head_argmax_no_finite_logits(hip_ctx):
    # d = +inf with nonzero scales makes every logit non-finite
    rows, cols = 3, 256
    b = bytearray(si_hip.synth_matrix(12, seed=3, rows=rows, cols=cols).tobytes())
    for r in range(rows):
        b[r * 144:r * 144 + 2] = struct.pack("<H", 0x7C00)
        b[r * 144 + 4:r * 144 + 16] = bytes([0x3F] * 12)
    H = hip_ctx.upload_quant_weight_private(bytes(b), 12)
    x = np.ones(cols, np.float32)
    with pytest.raises(si_hip.HipError) as e:
        hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x)
    assert e.value.status == -8
    tok, _ = hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x, rule=si_hip.ARGMAX_FIRST_GREATER)
    assert tok == O.argmax_first_greater(np.full(rows, np.nan, np.float32))


# ---- tensor rows, grouped submission, views, telemetry ---------------------------------
def test_tensor_rows_and_views(hip_ctx):
    rows, cols = 300, 1024
    w = si_hip.synth_matrix(14, seed=1300, rows=rows, cols=cols)
    x = si_hip.synth_normal(1301, cols)
    T = hip_ctx.upload_quant_weight_private(w, 14)
    full = hip_ctx.gguf_quant_matvec_weight(T, rows, cols, x)
    part = hip_ctx.gguf_quant_matvec_tensor_rows(T, (cols, rows), 37, 100, x)
    assert np.array_equal(part, full[37:137])
    with pytest.raises(si_hip.HipError) as e:
        hip_ctx.gguf_quant_matvec_tensor_rows(T, (cols, rows), 250, 51, x)
    assert e.value.status == -7 and e.value.message == "Q6_K row range is invalid"
    rb = cols // 256 * 210
    V = T.view(37 * rb, 100 * rb, 14)
    assert np.array_equal(hip_ctx.gguf_quant_matvec_weight(V, 100, cols, x), full[37:137])
    with pytest.raises(si_hip.HipError):
        T.view(0, rows * rb + 1, 14)


def test_grouped_matvecs_share_one_submission(hip_ctx):
    cols = 2048
    x = si_hip.synth_normal(1400, cols)
    specs = [(12, 64), (13, 33), (14, 100)]
    ws, raws = [], []
    for i, (t, r) in enumerate(specs):
        raw = si_hip.synth_matrix(t, seed=1401 + i, rows=r, cols=cols)
        raws.append(raw)
        ws.append(hip_ctx.upload_quant_weight_private(raw, t))
    before = hip_ctx.command_stats()
    outs = hip_ctx.gguf_quant_matvec_many_weights(ws, [r for _, r in specs], cols, x)
    after = hip_ctx.command_stats()
    assert after["waited"] - before["waited"] == 1
    # (one launch for the group; a lone matvec of the same matrix may take
    # another stage form, so the two agree within the bound)
    for (t, r), raw, y in zip(specs, raws, outs):
        _, y64, ab = O.matvec(t, raw, r, cols, x)
        assert_dot_close(y, y64, ab, what=f"grouped type {t}")
        assert_dot_close(hip_ctx.gguf_quant_matvec_weight(ws[specs.index((t, r))], r, cols, x),
                         y64, ab, what=f"lone type {t}")


def test_telemetry_counts_weights(hip_ctx):
    # weights of earlier tests held in reference cycles (a view and its
    # tensor) are freed by the cyclic collector, which may otherwise run in
    # the middle of this test's upload
    gc.collect()
    hip_ctx.reset_peaks()
    base = hip_ctx.current_allocated_bytes()
    w = si_hip.synth_matrix(12, seed=1500, rows=128, cols=1024)
    W = hip_ctx.upload_quant_weight_private(w, 12)
    assert hip_ctx.current_allocated_bytes() == base + w.size
    assert hip_ctx.peak_active_weight_bytes() >= w.size
    M = hip_ctx.bind_quant_weight_mapped(w, 12)
    assert M.is_mapped() and not W.is_mapped()
    assert W.byte_len() == w.size and W.ggml_type() == 12
    W.free()
    M.free()
    assert hip_ctx.current_allocated_bytes() == base
    assert hip_ctx.peak_allocated_bytes() >= base + w.size
    hip_ctx.reset_peaks()
    hip_ctx.sample_allocated()
    assert hip_ctx.peak_allocated_bytes() == hip_ctx.current_allocated_bytes() == base


def test_retained_errors_with_context(hip_ctx):
    w = si_hip.synth_matrix(12, seed=1600, rows=8, cols=512)
    W = hip_ctx.upload_quant_weight_private(w, 12)
    x = np.zeros(512, np.float32)
    with pytest.raises(si_hip.HipError) as e:
        hip_ctx.gguf_quant_matvec_weight(W, 9, 512, x)
    assert e.value.message == "Q4_K retained matvec byte length is invalid"
    with pytest.raises(si_hip.HipError) as e:
        hip_ctx.q4_k_fused_gate_up_weights(W, W, 8, 512, x[:256])
    assert e.value.message == "retained Q4_K fused gate/up dimensions are invalid"
    D = hip_ctx.upload_quant_weight_private(si_hip.synth_matrix(13, seed=1, rows=4, cols=256), 13)
    with pytest.raises(si_hip.HipError) as e:
        hip_ctx.gguf_quant_fused_mlp_weights(W, D, D, 8, 512, 4, x)
    assert e.value.message == "fused quantized MLP dimensions are invalid"


# ---- kernel structure probes ---------------------------------------------------------
@pytest.mark.parametrize("t", [12, 13, 14])
def test_matvec_unit_vectors_pick_each_column(hip_ctx, t):
    """x = e_k makes y[r] the dequantised weight w[r, k]: every column of every
    row must be read from the right place by the tuned kernels."""
    rows, cols = 67, 512
    w = si_hip.synth_matrix(t, seed=1700 + t, rows=rows, cols=cols)
    dq = O.dequantize(t, w, rows * cols).reshape(rows, cols)
    W = hip_ctx.upload_quant_weight_private(w, t)
    X = np.eye(cols, dtype=np.float32)
    bad = []
    for k in range(cols):
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, X[k])
        err = np.abs(y - dq[:, k])
        tol = 2e-5 * np.abs(dq[:, k]) + 1e-6
        if np.any(err > tol):
            bad.append((k, int(np.argmax(err - tol)), float(y[np.argmax(err - tol)]),
                        float(dq[np.argmax(err - tol), k])))
    cols_bad = sorted({b[0] for b in bad})
    assert bad == [], f"{len(bad)} columns wrong: {cols_bad}; first: {bad[:4]}"


# ---- captured submission (HIP graphs) ----------------------------------------------
def test_graph_replay_matches_eager(hip_ctx):
    """A decode-like sequence -- Q4_K matvec on a split launch (17408 x 5120),
    fused gate/up, Q6_K down, Q6_K head + argmax -- recorded once and replayed
    several times, with eager calls and synchronisations between the replays:
    every replay equals the eager run bit for bit, and the combine workspace is
    left clean (an eager split launch afterwards still matches)."""
    import ctypes as C
    lib = si_hip.lib()
    cols, rows, inter, vocab = 5120, 17408, 1024, 20011
    log("graph replay: building weights")
    wq = si_hip.synth_matrix(12, seed=3001, rows=rows, cols=cols, threads=8)
    wg = si_hip.synth_matrix(12, seed=3002, rows=inter, cols=cols, threads=8)
    wu = si_hip.synth_matrix(12, seed=3003, rows=inter, cols=cols, threads=8)
    wd = si_hip.synth_matrix(14, seed=3004, rows=cols, cols=inter, threads=8)
    wh = si_hip.synth_matrix(14, seed=3005, rows=vocab, cols=cols, threads=8)
    Wq, Wg, Wu, Wd, Wh = (hip_ctx.upload_quant_weight_private(w, t) for w, t in
                          ((wq, 12), (wg, 12), (wu, 12), (wd, 14), (wh, 14)))
    x = si_hip.synth_normal(3006, cols)
    d_x = hip_ctx.device_alloc(cols * 4)
    d_y = hip_ctx.device_alloc(rows * 4)
    d_h = hip_ctx.device_alloc(inter * 4)
    d_o = hip_ctx.device_alloc(cols * 4)
    d_l = hip_ctx.device_alloc(vocab * 4)
    d_r = hip_ctx.device_alloc(8)
    d_e = hip_ctx.device_alloc(cols * 4)  # eager work between replays
    hip_ctx.to_device(d_x, x)
    h = hip_ctx.handle
    P = C.c_void_p

    def enqueue():
        for rc in (
            lib.si_hip_quant_matvec_device(h, Wq.handle, rows, cols, P(d_x), P(d_y)),
            lib.si_hip_q4_k_fused_gate_up_device(h, Wg.handle, Wu.handle, inter, cols, P(d_x),
                                                 P(d_h)),
            lib.si_hip_quant_matvec_device(h, Wd.handle, cols, inter, P(d_h), P(d_o)),
            lib.si_hip_matvec_argmax_device(h, Wh.handle, vocab, cols, P(d_x),
                                            si_hip.ARGMAX_LAST_FINITE, P(d_l), P(d_r)),
        ):
            assert rc == 0, si_hip.last_error()

    def results():
        hip_ctx.synchronize()
        return (hip_ctx.from_device(d_y, rows), hip_ctx.from_device(d_h, inter),
                hip_ctx.from_device(d_o, cols), hip_ctx.from_device(d_l, vocab),
                hip_ctx.from_device(d_r, 1, np.uint64))

    def clear():
        for p, n in ((d_y, rows), (d_h, inter), (d_o, cols), (d_l, vocab)):
            hip_ctx.to_device(p, np.full(n, np.nan, np.float32))
        hip_ctx.to_device(d_r, np.zeros(1, np.uint64))

    enqueue()
    ref = results()
    _, y64, ab = O.matvec(12, wq, rows, cols, x, threads=8)
    assert_dot_close(ref[0], y64, ab, what="eager split matvec")

    log("graph replay: capture")
    hip_ctx.capture_begin()
    enqueue()
    graph = hip_ctx.capture_end()
    assert graph.calls == 4
    for rep in range(3):
        clear()
        # eager work on the same context between replays
        assert lib.si_hip_quant_matvec_device(h, Wd.handle, cols, inter, P(d_h), P(d_e)) == 0
        hip_ctx.synchronize()
        log(f"graph replay {rep}")
        graph.launch()
        got = results()
        for a, b in zip(got[:4], ref[:4]):
            assert same_bits(a, b), f"replay {rep} differs"
        assert got[4][0] == ref[4][0]
    graph.free()
    clear()
    enqueue()
    again = results()
    for a, b in zip(again[:4], ref[:4]):
        assert same_bits(a, b)
    for p in (d_x, d_y, d_h, d_o, d_l, d_r, d_e):
        hip_ctx.device_free(p)


@pytest.mark.parametrize("t", [12, 13, 14])
def test_graph_replay_matmul_many_groups(hip_ctx, t):
    """Multi-token verify on the vectors-in-rows path (a K-sliced launch whose
    stage or slice sums a second kernel adds up; Q4_K, Q5_K and Q6_K): 3, 8
    and 16 vectors recorded in one graph, replayed with other launches of the
    same workspace in between, bit for bit equal to the eager calls and to the
    oracle's bound."""
    import ctypes as C
    lib = si_hip.lib()
    rows, cols = 1040, 5120
    w = si_hip.synth_matrix(t, seed=3101 + t, rows=rows, cols=cols, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, t)
    X = si_hip.synth_normal(3102, 16 * cols).reshape(16, cols)
    d_x = hip_ctx.device_alloc(16 * cols * 4)
    hip_ctx.to_device(d_x, X)
    outs = {m: hip_ctx.device_alloc(m * rows * 4) for m in (3, 8, 16)}
    d_e = hip_ctx.device_alloc(4 * rows * 4)
    h, P = hip_ctx.handle, C.c_void_p

    def enqueue():
        for m, d in outs.items():
            assert lib.si_hip_matmul_many_device(h, W.handle, rows, cols, m, P(d_x), P(d)) == 0, \
                si_hip.last_error()

    def results():
        hip_ctx.synchronize()
        return {m: hip_ctx.from_device(d, m * rows).reshape(m, rows) for m, d in outs.items()}

    enqueue()
    ref = results()
    for b in range(16):
        _, y64, ab = O.matvec(t, w, rows, cols, X[b], threads=8)
        assert_dot_close(ref[16][b], y64, ab, what=f"eager vector {b}")
        if b < 3:
            assert_dot_close(ref[3][b], y64, ab, what=f"eager vector {b} of 3")
        if b < 8:
            assert_dot_close(ref[8][b], y64, ab, what=f"eager vector {b} of 8")
    hip_ctx.capture_begin()
    enqueue()
    graph = hip_ctx.capture_end()
    for rep in range(3):
        for m, d in outs.items():
            hip_ctx.to_device(d, np.full(m * rows, np.nan, np.float32))
        # another grouped launch on the same scratch between replays
        assert lib.si_hip_matmul_many_device(h, W.handle, rows, cols, 4, P(d_x), P(d_e)) == 0
        hip_ctx.synchronize()
        graph.launch()
        got = results()
        for m in outs:
            assert same_bits(got[m], ref[m]), f"replay {rep}, {m} vectors"
    graph.free()
    for d in list(outs.values()) + [d_x, d_e]:
        hip_ctx.device_free(d)


def test_graph_capture_state_errors(hip_ctx):
    with pytest.raises(si_hip.HipError):
        hip_ctx.capture_end()
    hip_ctx.capture_begin()
    try:
        with pytest.raises(si_hip.HipError):
            hip_ctx.capture_begin()
    finally:
        g = hip_ctx.capture_end()
    assert g.calls == 0
    g.free()
