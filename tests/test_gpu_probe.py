"""GPU: the measurement probe (si_hip_stream_probe) runs every mode on Q4_K
and Q5_K weights and rejects what it does not read.  It computes nothing;
its use is the timing in bench.py."""
import ctypes as C

import pytest

import si_hip

pytestmark = pytest.mark.gpu


def _probe(ctx, weights, rows, cols, mode, iters=3):
    harr = (C.c_void_p * len(weights))(*[w.handle.value for w in weights])
    return si_hip.lib().si_hip_stream_probe(ctx.handle, harr, len(weights), rows, cols, mode,
                                            iters)


@pytest.mark.parametrize("t", [12, 13])
def test_probe_modes(hip_ctx, t):
    rows, cols = 1000, 5120  # a partial last tile
    W = [hip_ctx.upload_quant_weight_private(si_hip.synth_matrix(t, seed=9000 + i, rows=rows,
                                                                 cols=cols), t) for i in range(2)]
    try:
        for mode in (0, 1, 2, 3):
            assert _probe(hip_ctx, W, rows, cols, mode) == 0, si_hip.last_error()
        for mode in (4, 5, 6):  # Q4_K only
            assert _probe(hip_ctx, W, rows, cols, mode) == (0 if t == 12 else -5)
        hip_ctx.synchronize()
        assert _probe(hip_ctx, W, rows, cols, 7) == -7
        assert _probe(hip_ctx, W, rows, cols + 256, 0) != 0  # byte length mismatch
        if t == 12:  # full-line copies need rows of 4 mod 8 blocks
            V = [hip_ctx.upload_quant_weight_private(
                si_hip.synth_matrix(t, seed=9010, rows=64, cols=4096), t)]
            try:
                assert _probe(hip_ctx, V, 64, 4096, 4) == -2
                assert _probe(hip_ctx, V, 64, 4096, 5) == 0, si_hip.last_error()
                hip_ctx.synchronize()
            finally:
                V[0].free()
    finally:
        for w in W:
            w.free()


def test_probe_rejects_q6k(hip_ctx):
    W = hip_ctx.upload_quant_weight_private(si_hip.synth_matrix(14, seed=9100, rows=64,
                                                                cols=512), 14)
    try:
        assert _probe(hip_ctx, [W], 64, 512, 0) == -5
    finally:
        W.free()
