"""GPU: the fused MLP (gguf_quant_fused_mlp_weights, metal.rs:3569-3732) is
the fused gate/up (q4_k_fused_gate_up, metal.rs:498-587) into h followed by
the down matvec of h (metal.rs:895-1050), bit for bit, through the host and
the device entry points, three calls in a row (the kernels' tile counters
must be back at zero after every call); and within the chain's bound of the
oracle (quant.rs per-weight values).
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
import si_hip
from test_gpu_parity import DOT_TOL, gate_up_bound, same_bits, silu64

pytestmark = pytest.mark.gpu

Q4, Q6 = 12, 14


def log(msg):
    print(msg, flush=True)


def _mlp_case(hip_ctx, gate_rows, cols, seed, x):
    down_rows = cols
    gw = si_hip.synth_matrix(Q4, seed=seed, rows=gate_rows, cols=cols, threads=8)
    uw = si_hip.synth_matrix(Q4, seed=seed + 1, rows=gate_rows, cols=cols, threads=8)
    dw = si_hip.synth_matrix(Q6, seed=seed + 2, rows=down_rows, cols=gate_rows, threads=8)
    W = [hip_ctx.upload_quant_weight_private(gw, Q4), hip_ctx.upload_quant_weight_private(uw, Q4),
         hip_ctx.upload_quant_weight_private(dw, Q6)]
    return (gw, uw, dw), W, down_rows


# (gate rows, K): the 17408 x 5120 gate/up with its 5120 x 17408 down
# projection, a short one, and one whose rows are of 0 mod 8 blocks (the
# gate/up kernel then copies 64-byte pieces, not whole lines)
@pytest.mark.parametrize("gate_rows,cols", [(17408, 5120), (2048, 1024), (4096, 4096)])
def test_fused_mlp_equals_two_launches(hip_ctx, gate_rows, cols):
    log(f"fused MLP chain {gate_rows}x{cols}")
    x = si_hip.synth_normal(gate_rows + cols, cols, scale=0.1)
    (gw, uw, dw), (G, U, D), down_rows = _mlp_case(hip_ctx, gate_rows, cols, 6100, x)
    try:
        h = hip_ctx.q4_k_fused_gate_up_weights(G, U, gate_rows, cols, x)
        y_two = hip_ctx.gguf_quant_matvec_weight(D, down_rows, gate_rows, h)
        for rep in range(3):
            y = hip_ctx.gguf_quant_fused_mlp_weights(G, U, D, gate_rows, cols, down_rows, x)
            assert same_bits(y, y_two), f"call {rep}"
        # the device entry point, three calls in a row
        lib = si_hip.lib()
        d_x = hip_ctx.device_alloc(cols * 4)
        d_h = hip_ctx.device_alloc(gate_rows * 4)
        d_y = hip_ctx.device_alloc(down_rows * 4)
        try:
            hip_ctx.to_device(d_x, x)
            for rep in range(3):
                rc = lib.si_hip_fused_mlp_device(hip_ctx.handle, G.handle, U.handle, D.handle,
                                                 gate_rows, cols, down_rows, C.c_void_p(d_x),
                                                 C.c_void_p(d_h), C.c_void_p(d_y))
                assert rc == 0, si_hip.last_error()
                hip_ctx.synchronize()
                assert same_bits(hip_ctx.from_device(d_h, (gate_rows,)), h), f"h, call {rep}"
                assert same_bits(hip_ctx.from_device(d_y, (down_rows,)), y_two), f"y, call {rep}"
        finally:
            for p in (d_x, d_h, d_y):
                hip_ctx.device_free(p)
        # and the oracle's bound
        _, g64, ag = O.matvec(Q4, gw, gate_rows, cols, x, threads=16)
        _, u64, au = O.matvec(Q4, uw, gate_rows, cols, x, threads=16)
        h64 = silu64(g64) * u64
        hb = gate_up_bound(g64, ag, u64, au)
        wd = O.dequantize(Q6, dw, down_rows * gate_rows).reshape(down_rows, gate_rows)
        wd = wd.astype(np.float64)
        bound = DOT_TOL * (np.abs(wd) @ np.abs(h64)) + np.abs(wd) @ hb + 1e-30
        assert np.all(np.abs(y_two - wd @ h64) <= bound)
    finally:
        for w in (G, U, D):
            w.free()


def test_fused_mlp_chain_special_activations(hip_ctx):
    """Activations that make h non-finite (the down projection takes its exact
    path) and tiny (blocks whose digits round): still bit for bit the two
    launches."""
    gate_rows, cols = 17408, 5120
    log("fused MLP chain, special activations")
    x = si_hip.synth_normal(6200, cols, scale=0.1)
    x[17] = np.inf          # every gate/up row: +-inf or NaN
    (gw, uw, dw), (G, U, D), down_rows = _mlp_case(hip_ctx, gate_rows, cols, 6201, x)
    x2 = si_hip.synth_normal(6202, cols, scale=1e-6)
    try:
        for xx in (x, x2):
            h = hip_ctx.q4_k_fused_gate_up_weights(G, U, gate_rows, cols, xx)
            y_two = hip_ctx.gguf_quant_matvec_weight(D, down_rows, gate_rows, h)
            y = hip_ctx.gguf_quant_fused_mlp_weights(G, U, D, gate_rows, cols, down_rows, xx)
            assert same_bits(y, y_two)
    finally:
        for w in (G, U, D):
            w.free()
