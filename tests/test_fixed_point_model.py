"""CPU model of the matrix-core kernels' activation handling (no GPU).

The kernels (memory-aware-inference_amd/csrc/mfma_common.h, split_chunk,
build_images, rounded_redo; side_list in the vectors-in-rows kernel) write
each 256-element block of x as X * 2^(e - 30), X an integer of at most 30
bits and e the exponent of the block's largest |x| (largest |x| < 2^e).
Non-zero activations below 2^(e - 14) are "side" elements:

  * up to side_max of them in a block: left out of X and added back with
    exact per-weight products ("side" blocks).  side_max is 8 in the
    vectors-in-rows kernel (q4k_tokens_mfma) and 0 in the others;
  * more: kept in X, rounded like the rest ("rounded" blocks).  Per row and
    stage the kernel bounds their rounding error by (largest |w| of the
    lane's 64-element share) x (sum of the side elements' |rounding error|
    in that share), and compares it with the sum of the shares' |partial
    dot|; a row that fails recomputes its rounded blocks exactly.

A block with a non-finite or huge activation takes the exact path.  This
model restates those rules in numpy and measures the error they leave against
the f64 dot.  Elements kept in X have relative error at most 2^-17, and the
rounded blocks at most kRoundedTol = 4e-6 of sum|w*x|, so the activation
rounding stays below (2^-17 + 4e-6) * sum|w*x|, 0.58 of the 2e-5 bar, whatever
the weights.  The rule the kernels used before (a block goes exact only when a
whole 16-element chunk lies 2^13 below the block maximum) is modelled too, to
show that the crafted input does catch it.
"""
import numpy as np
import pytest

import crafted
import oracle_lib as O
import si_hip

BAR = 2e-5
SIDE_SHIFT = 14
SIDE_MAX_TOKENS = 8  # q4k_tokens_mfma lists up to 8 side elements of a block
SIDE_MAX_MATVEC = 0  # the other matrix-core kernels round every side block
SIDE_MAXES = [SIDE_MAX_MATVEC, SIDE_MAX_TOKENS]
TOL = 4e-6
LIMIT = (2.0 ** -17 + TOL) / BAR  # 0.58


def _block_split(v, side_max=SIDE_MAX_MATVEC):
    """(kind, fixed-point x) of one block, kind in fixed/side/rounded/exact."""
    a = np.abs(v)
    if not (np.all(np.isfinite(v)) and np.all(a < 2.0 ** 100)):
        return "exact", v
    e = int(np.frexp(float(a.max()))[1])  # largest |x| < 2^e
    fixed = np.rint(np.ldexp(v, 30 - e)) * 2.0 ** (e - 30)
    side = (v != 0) & (a < 2.0 ** (e - SIDE_SHIFT))
    if not side.any():
        return "fixed", fixed
    if side.sum() <= side_max:
        return "side", np.where(side, v, fixed)
    return "rounded", fixed


def model_dot(w, x, rule="side", side_max=SIDE_MAX_MATVEC, stage=4):
    """The kernel's activation handling for every row of w: returns
    (y as the kernel would compute it in exact arithmetic, per-block kinds,
    number of row-stages that recompute their rounded blocks)."""
    x64 = np.asarray(x, np.float32).astype(np.float64)
    nb = x64.size // 256
    xb = x64.reshape(nb, 256)
    kinds, xe = [], np.empty_like(xb)
    for b in range(nb):
        if rule == "side":
            k, f = _block_split(xb[b], side_max)
        else:  # the chunk rule
            v = xb[b]
            a = np.abs(v)
            amax = float(a.max())
            e = int(np.frexp(amax)[1])
            cmax = a.reshape(16, 16).max(axis=1)
            bad = not np.all(np.isfinite(v)) or np.any((cmax > 0) & (cmax < amax * 2.0 ** -13))
            k, f = ("exact", v) if bad else ("fixed", np.rint(np.ldexp(v, 30 - e)) * 2.0 ** (e - 30))
        kinds.append(k)
        xe[b] = f
    rows = w.shape[0]
    wb = w.reshape(rows, nb, 256)
    # per row, block and 64-element share: the dot with the kernel's x
    shares = np.einsum("rbgk,bgk->rbg", wb.reshape(rows, nb, 4, 64), xe.reshape(nb, 4, 64))
    y = shares.sum(axis=(1, 2))
    redone = 0
    rounded = [b for b, k in enumerate(kinds) if k == "rounded"]
    for s0 in range(0, nb, stage):
        blocks = [b for b in rounded if s0 <= b < s0 + stage]
        if not blocks:
            continue
        # error bound of each row: max |w| of the share x its side-error sum
        err = np.zeros(rows)
        for b in blocks:
            v = xb[b]
            e = int(np.frexp(float(np.abs(v).max()))[1])
            side = (v != 0) & (np.abs(v) < 2.0 ** (e - SIDE_SHIFT))
            serr = (np.abs(v - xe[b]) * side).reshape(4, 64).sum(axis=1)  # per share
            wmax = np.abs(wb[:, b, :]).reshape(rows, 4, 64).max(axis=2)
            err += (wmax * serr).sum(axis=1)
        a = np.abs(shares[:, s0:s0 + stage, :]).sum(axis=(1, 2))
        fail = ~(err * 1.01 <= TOL * (a - err))
        redone += int(fail.sum())
        for b in blocks:  # the failing rows' rounded blocks, exactly
            y[fail] += wb[fail, b, :] @ (xb[b] - xe[b])
    return y, kinds, redone


def error_ratio(w, x, rule="side", side_max=SIDE_MAX_MATVEC, stage=4):
    y, _, _ = model_dot(w, x, rule, side_max, stage)
    x64 = np.asarray(x, np.float32).astype(np.float64)
    err = np.abs(y - w @ x64)
    return float(np.max(err / (BAR * (np.abs(w) @ np.abs(x64)))))


def _weights(t, rows, cols, seed):
    raw = crafted.zero_weight_matrix(t, rows, cols, seed)
    w = O.dequantize(t, raw, rows * cols).reshape(rows, cols).astype(np.float64)
    assert np.all(w.reshape(rows, -1, 256)[:, :, crafted.ZERO_ELEMS] == 0.0)
    return w


@pytest.mark.parametrize("t", [12, 13, 14])
def test_crafted_weights_are_zero_where_asked(t):
    _weights(t, 8, 1024, 5 + t)


@pytest.mark.parametrize("side_max,stage", [(0, 4), (0, 2), (8, 4)])
@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("case", crafted.CASES)
def test_side_rule_meets_the_bar_on_crafted_inputs(t, case, side_max, stage):
    rows, cols = 24, 2048
    w = _weights(t, rows, cols, 40 + t)
    x = crafted.crafted_x(cols, case, 7 + t)
    ratio = error_ratio(w, x, side_max=side_max, stage=stage)
    assert ratio <= LIMIT, f"{case}: {ratio:.3g} of the bar"


def test_chunk_rule_fails_the_crafted_input():
    """The crafted "tiny" input is the case the chunk rule let through."""
    w = _weights(14, 24, 2048, 77)
    x = crafted.crafted_x(2048, "tiny", 78)
    assert error_ratio(w, x, "chunk") > 10.0
    assert error_ratio(w, x) <= LIMIT


def test_crafted_tiny_blocks_are_rounded_and_redone():
    """All small activations on the weights: every rounded block fails the
    check (its error bound is large against its own dot) and is redone."""
    w = _weights(12, 16, 1024, 3)
    y, kinds, redone = model_dot(w, crafted.crafted_x(1024, "tiny", 3))
    assert kinds == ["rounded"] * 4
    assert redone == 16


def test_crafted_many_blocks_are_rounded_and_pass():
    w = _weights(13, 16, 2048, 4)
    y, kinds, redone = model_dot(w, crafted.crafted_x(2048, "many", 4))
    assert kinds == ["rounded"] * 8
    assert redone == 0


def test_side_rule_routes_crafted_blocks():
    w = np.ones((2, 9 * 256))
    x = crafted.crafted_x(9 * 256, "side", 3)
    _, kinds, _ = model_dot(w, x, side_max=SIDE_MAX_TOKENS)
    assert kinds == ["side"] * 9  # 1..8 side elements per block, all listed
    _, kinds, redone = model_dot(w, x)
    assert kinds == ["rounded"] * 9 and redone == 0  # the same blocks rounded pass
    _, kinds, _ = model_dot(w[:, :512], crafted.crafted_x(2 * 256, "edge", 3))
    assert kinds == ["fixed", "fixed"]


def test_side_elements_are_rare_on_normal_activations():
    """Share of N(0,1) blocks with side elements, over 20,000 blocks: listed
    in the vectors-in-rows kernel (more than its list holds: rounded), rounded
    in the others, whose rows then pass the check on random weights."""
    x = si_hip.synth_normal(12345, 20000 * 256)
    blocks = x.astype(np.float64).reshape(-1, 256)
    kinds = [_block_split(v, SIDE_MAX_TOKENS)[0] for v in blocks]
    side = kinds.count("side") / len(kinds)
    rounded = kinds.count("rounded") / len(kinds)
    print(f"N(0,1) blocks: {side:.4f} with side elements, {rounded:.6f} past the list")
    assert 0.0 < side < 0.1
    assert rounded < 1e-4
    assert [_block_split(v)[0] for v in blocks].count("rounded") / len(kinds) == side
    raw = si_hip.synth_matrix(12, seed=11, rows=64, cols=64 * 256)
    w = O.dequantize(12, raw, 64 * 64 * 256).reshape(64, -1).astype(np.float64)
    for stage in (4, 2):
        _, kinds, redone = model_dot(w, x[:64 * 256], stage=stage)
        assert "rounded" in kinds and redone == 0


def test_swiglu_intermediate_is_rounded_not_redone():
    """h = silu(g) * u of large random projections: half of h is many orders
    of magnitude below the block maximum, so every block is rounded; the
    check passes on the rows (the bound is tiny against the dot)."""
    rng = np.random.default_rng(9)
    g = rng.normal(0, 35, 4096)
    u = rng.normal(0, 35, 4096)
    h = (g / (1 + np.exp(-g)) * u).astype(np.float32)
    raw = si_hip.synth_matrix(14, seed=10, rows=64, cols=4096)
    w = O.dequantize(14, raw, 64 * 4096).reshape(64, 4096).astype(np.float64)
    y, kinds, redone = model_dot(w, h)
    assert kinds.count("rounded") >= 14
    assert redone == 0
    assert error_ratio(w, h) <= LIMIT


@pytest.mark.parametrize("side_max", SIDE_MAXES)
@pytest.mark.parametrize("seed", range(3))
def test_side_rule_on_heavy_tailed_activations(seed, side_max):
    """Student-t activations with a few massive channels (the shape of real
    decoder activations) on random Q4_K weights."""
    rows, cols = 32, 4096
    raw = si_hip.synth_matrix(12, seed=seed, rows=rows, cols=cols)
    w = O.dequantize(12, raw, rows * cols).reshape(rows, cols).astype(np.float64)
    rng = np.random.default_rng(seed)
    x = rng.standard_t(2.0, cols)
    x[rng.choice(cols, 6, replace=False)] *= 1e4
    assert error_ratio(w, x.astype(np.float32), side_max=side_max) <= LIMIT
