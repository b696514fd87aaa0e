"""GPU: the matrix-core kernels' fixed-point activations against the oracle on
inputs built to defeat them (tests/crafted.py): small activations carrying the
whole dot next to large ones on zero weights, side lists of 1..5 entries per
block, and activations just above the side threshold.  Every dot must stay
within 2e-5 * sum|w*x| of the f64 value of the exact products (quant.rs
weights), through every kernel that builds digit images: Q4_K/Q5_K/Q6_K at
M = 1 (including the 17408-column down projection), fused gate/up, the fused
MLP, matmul-many at M = 4 and 16, the grouped launch and the output head with
its argmax, under the default and the generic kernel policy.
"""
import numpy as np
import pytest

import crafted
import oracle_lib as O
import si_hip
from test_gpu_parity import assert_dot_close, gate_up_bound, log, silu64

pytestmark = pytest.mark.gpu

POLICIES = [si_hip.KERNEL_AUTO, si_hip.KERNEL_GENERIC]


@pytest.fixture(params=POLICIES, ids=["auto", "generic"])
def ctx(request, hip_ctx):
    hip_ctx.set_kernel_policy(request.param)
    yield hip_ctx
    hip_ctx.set_kernel_policy(si_hip.KERNEL_AUTO)


@pytest.mark.parametrize("case", crafted.CASES)
@pytest.mark.parametrize("t,rows,cols", [(12, 160, 5120), (13, 160, 5120), (14, 160, 5120),
                                         (12, 40, 17408), (14, 96, 17408), (12, 17408, 5120)])
def test_crafted_matvec(ctx, case, t, rows, cols):
    log(f"crafted matvec {case} t={t} {rows}x{cols}")
    w = crafted.zero_weight_matrix(t, rows, cols, seed=rows + cols + t)
    x = crafted.crafted_x(cols, case, seed=cols + t)
    _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
    W = ctx.upload_quant_weight_private(w, t)
    y = ctx.gguf_quant_matvec_weight(W, rows, cols, x)
    assert_dot_close(y, y64, ab, what=f"{case} type {t} {rows}x{cols}")


@pytest.mark.parametrize("case", crafted.CASES)
def test_crafted_fused_gate_up(ctx, case):
    rows, cols = 1000, 5120
    log(f"crafted gate/up {case}")
    gw = crafted.zero_weight_matrix(12, rows, cols, seed=11)
    uw = crafted.zero_weight_matrix(12, rows, cols, seed=12)
    x = crafted.crafted_x(cols, case, seed=13)
    _, g64, ag = O.matvec(12, gw, rows, cols, x, threads=8)
    _, u64, au = O.matvec(12, uw, rows, cols, x, threads=8)
    G = ctx.upload_quant_weight_private(gw, 12)
    U = ctx.upload_quant_weight_private(uw, 12)
    h = ctx.q4_k_fused_gate_up_weights(G, U, rows, cols, x)
    err = np.abs(h.astype(np.float64) - silu64(g64) * u64)
    assert np.all(err <= gate_up_bound(g64, ag, u64, au))


@pytest.mark.parametrize("case", crafted.CASES)
def test_crafted_fused_mlp(ctx, case):
    gate_rows, cols, down_rows = 2048, 1024, 512
    log(f"crafted mlp {case}")
    gw = crafted.zero_weight_matrix(12, gate_rows, cols, seed=21)
    uw = crafted.zero_weight_matrix(12, gate_rows, cols, seed=22)
    dw = crafted.zero_weight_matrix(14, down_rows, gate_rows, seed=23)
    x = crafted.crafted_x(cols, case, seed=24)
    _, g64, ag = O.matvec(12, gw, gate_rows, cols, x, threads=8)
    _, u64, au = O.matvec(12, uw, gate_rows, cols, x, threads=8)
    h64 = silu64(g64) * u64
    hb = gate_up_bound(g64, ag, u64, au)
    wd = O.dequantize(14, dw, down_rows * gate_rows).reshape(down_rows, gate_rows)
    wd = wd.astype(np.float64)
    y64 = wd @ h64
    bound = 2e-5 * (np.abs(wd) @ np.abs(h64)) + np.abs(wd) @ hb + 1e-30
    G = ctx.upload_quant_weight_private(gw, 12)
    U = ctx.upload_quant_weight_private(uw, 12)
    D = ctx.upload_quant_weight_private(dw, 14)
    y = ctx.gguf_quant_fused_mlp_weights(G, U, D, gate_rows, cols, down_rows, x)
    assert np.all(np.abs(y - y64) <= bound)


@pytest.mark.parametrize("batch", [4, 16])
@pytest.mark.parametrize("t", [12, 13, 14])
def test_crafted_matmul_many(ctx, t, batch):
    rows, cols = 300, 5120
    log(f"crafted matmul_many t={t} batch={batch}")
    w = crafted.zero_weight_matrix(t, rows, cols, seed=31 + t)
    X = np.stack([crafted.crafted_x(cols, crafted.CASES[b % 3], seed=100 + b)
                  if b % 4 != 3 else si_hip.synth_normal(100 + b, cols)
                  for b in range(batch)])
    W = ctx.upload_quant_weight_private(w, t)
    outs = ctx.gguf_quant_matmul_many_weight(W, rows, cols, batch, X)
    for b in range(batch):
        _, y64, ab = O.matvec(t, w, rows, cols, X[b], threads=8)
        assert_dot_close(outs[b], y64, ab, what=f"type {t} candidate {b}")


@pytest.mark.parametrize("t", [12, 14])
def test_crafted_grouped_matvec(hip_ctx, t):
    rows, cols = [512, 128, 130], 5120
    log(f"crafted grouped t={t}")
    ws = [crafted.zero_weight_matrix(t, r, cols, seed=41 + k) for k, r in enumerate(rows)]
    x = crafted.crafted_x(cols, "side", seed=44)
    Ws = [hip_ctx.upload_quant_weight_private(w, t) for w in ws]
    outs = hip_ctx.gguf_quant_matvec_many_weights(Ws, rows, cols, x)
    for w, r, y in zip(ws, rows, outs):
        _, y64, ab = O.matvec(t, w, r, cols, x, threads=8)
        assert_dot_close(y, y64, ab, what=f"grouped type {t} rows {r}")


@pytest.mark.parametrize("case", crafted.CASES)
def test_crafted_head_argmax(ctx, case):
    vocab, cols = 20011, 5120
    log(f"crafted head {case}")
    head = crafted.zero_weight_matrix(14, vocab, cols, seed=51)
    x = crafted.crafted_x(cols, case, seed=52)
    H = ctx.upload_quant_weight_private(head, 14)
    token, logits = ctx.gguf_quant_matvec_argmax_weight(H, vocab, cols, x)
    y32, y64, ab = O.matvec(14, head, vocab, cols, x, threads=8)
    assert_dot_close(logits, y64, ab, what=f"head {case}")
    top2 = np.sort(y64)[-2:]
    if top2[1] - top2[0] > 4e-5 * ab.max():
        assert token == int(np.argmax(y64))
    assert token == int(np.argmax(logits))
