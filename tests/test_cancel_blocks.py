"""The cancelling-block generator (tests/cancel_blocks.py) against the oracle's
dequantisation (quant.rs restated): rows of kind 0 decode to all zeros, kind 1
and 2 rows to mostly zeros, so the GPU tests that use them do exercise weights
that cancel inside their own decode.  No GPU."""
import numpy as np
import pytest

import cancel_blocks as CB
import oracle_lib as O


@pytest.mark.parametrize("t", [CB.Q4, CB.Q5])
def test_generated_weights_cancel(t):
    rows, cols = 64, 2048
    w = CB.matrix(t, rows, cols, seed=5)
    deq = O.dequantize(t, w, rows * cols).reshape(rows, cols)
    kinds = CB.row_kinds(rows)
    zero = (deq == 0.0).mean(axis=1)
    assert np.all(zero[kinds == 0] == 1.0)             # every weight exactly 0
    assert np.all(zero[kinds == 1] > 0.97)             # ~99 % cancel
    assert np.all((zero[kinds == 2] > 0.8) & (zero[kinds == 2] < 0.99))
    assert np.all(zero[kinds == 3] < 0.2)              # ordinary rows
    # the two products are large where they cancel: the min term is far from 0
    d = np.frombuffer(w, np.uint8).reshape(rows, cols // 256, -1)[:, :, 0:2].copy()
    assert np.all(d.view(np.float16) > 0)


def test_oracle_dot_of_cancelling_rows_is_zero():
    rows, cols = 8, 1024
    w = CB.matrix(CB.Q4, rows, cols, seed=9)
    x = np.random.default_rng(1).normal(size=cols).astype(np.float32)
    y32, y64, ab = O.matvec(CB.Q4, w, rows, cols, x)
    k0 = CB.row_kinds(rows) == 0
    assert np.all(y32[k0] == 0.0) and np.all(y64[k0] == 0.0) and np.all(ab[k0] == 0.0)
    # (a row of kind 1 may have no changed quant at this size and cancel whole)
    assert np.all(ab[CB.row_kinds(rows) >= 2] > 0.0)
