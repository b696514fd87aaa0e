"""GPU: every BASELINE.json config at its full size against the oracle.

  1  Q4_K 4096 x 5120 (the CPU reference's matrix)
  3  fused SwiGLU MLP: gate/up Q4_K 17408 x 5120 -> down Q6_K 5120 x 17408,
     x ~ N(0,1) * 0.1, as one chained call
  4  Q5_K 5120 x 5120; the Q6_K head 151936 x 5120 + greedy argmax (both tie
     rules, top-2 margin reported); the chained Q5_K -> head; 64 Q4_K
     embedding rows from the 151936 x 5120 table
  5  matmul-many on Q4_K 17408 x 5120 for M = 2, 4, 8, 16; the 64-layer
     aggregate's per-layer shapes, and one token of it through the device
     calls against the host calls, bit for bit

Bars: dots within 2e-5 * sum|w*x| of the f64 value of
the exact products; embedding rows bit-exact; argmax identical.  Weights come
from the seeded generator (si_hip.synth_*), whose distributions are the
configs' (d, dmin ~ |N(0, 0.02)|, random scale and quant bytes; Q6_K scales
uniform in [-32, 31], d ~ |N(0, 0.01)|).
"""
import numpy as np
import pytest

import oracle_lib as O
import si_hip
from test_gpu_parity import assert_dot_close, gate_up_bound, log, silu64

pytestmark = pytest.mark.gpu

Q4, Q5, Q6 = 12, 13, 14
VOCAB, K, N = 151936, 5120, 17408


@pytest.fixture(scope="module")
def head(hip_ctx):
    w = si_hip.synth_matrix(Q6, seed=4001, rows=VOCAB, cols=K, threads=16)
    H = hip_ctx.upload_quant_weight_private(w, Q6)
    yield w, H
    H.free()


def test_config1_q4k_4096x5120(hip_ctx):
    rows, cols = 4096, 5120
    w = si_hip.synth_matrix(Q4, seed=1, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(2, cols)
    y32, y64, ab = O.matvec(Q4, w, rows, cols, x, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, Q4)
    y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
    worst = assert_dot_close(y, y64, ab, what="config 1")
    ref_worst = float(np.max(np.abs(y32.astype(np.float64) - y64) / (2e-5 * ab)))
    log(f"config 1: GPU worst {worst:.4f} of the bar; the reference's sequential f32 dot "
        f"{ref_worst:.4f}")


def test_config3_chained_mlp_full_size(hip_ctx):
    log("config 3: fused MLP 17408 x 5120 -> 5120 x 17408")
    gw = si_hip.synth_matrix(Q4, seed=3001, rows=N, cols=K, threads=16)
    uw = si_hip.synth_matrix(Q4, seed=3002, rows=N, cols=K, threads=16)
    dw = si_hip.synth_matrix(Q6, seed=3003, rows=K, cols=N, threads=16)
    x = si_hip.synth_normal(3004, K, scale=0.1)
    _, g64, ag = O.matvec(Q4, gw, N, K, x, threads=16)
    _, u64, au = O.matvec(Q4, uw, N, K, x, threads=16)
    h64 = silu64(g64) * u64
    hb = gate_up_bound(g64, ag, u64, au)
    wd = O.dequantize(Q6, dw, K * N).reshape(K, N).astype(np.float64)
    y64 = wd @ h64
    awd = np.abs(wd)
    bound = 2e-5 * (awd @ np.abs(h64)) + awd @ hb + 1e-30
    G = hip_ctx.upload_quant_weight_private(gw, Q4)
    U = hip_ctx.upload_quant_weight_private(uw, Q4)
    D = hip_ctx.upload_quant_weight_private(dw, Q6)
    y = hip_ctx.gguf_quant_fused_mlp_weights(G, U, D, N, K, K, x)
    ratio = np.abs(y - y64) / bound
    log(f"  worst error / bound {ratio.max():.4f}")
    assert np.all(ratio <= 1.0)
    # the same chain one call at a time: gate/up, then the down matvec on h
    h = hip_ctx.q4_k_fused_gate_up_weights(G, U, N, K, x)
    y2 = hip_ctx.gguf_quant_matvec_weight(D, K, N, h)
    assert np.array_equal(y, y2)


def test_config4_q5k_5120x5120(hip_ctx):
    w = si_hip.synth_matrix(Q5, seed=4101, rows=5120, cols=K, threads=8)
    x = si_hip.synth_normal(4102, K)
    _, y64, ab = O.matvec(Q5, w, 5120, K, x, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, Q5)
    assert_dot_close(hip_ctx.gguf_quant_matvec_weight(W, 5120, K, x), y64, ab, what="Q5_K 5120^2")


def _head_check(hip_ctx, w, H, x, what):
    tok, logits = hip_ctx.gguf_quant_matvec_argmax_weight(H, VOCAB, K, x)
    y32, y64, ab = O.matvec(Q6, w, VOCAB, K, x, threads=16)
    assert_dot_close(logits, y64, ab, what=what)
    order = np.argsort(y64)
    top, second = int(order[-1]), int(order[-2])
    margin = y64[top] - y64[second]
    log(f"{what}: token {tok}, top-2 margin {margin:.6g} (error bound "
        f"{2e-5 * (ab[top] + ab[second]):.3g})")
    assert margin > 2e-5 * (ab[top] + ab[second])
    assert tok == top == O.argmax_last_finite(y32)
    first, _ = hip_ctx.gguf_quant_matvec_argmax_weight(H, VOCAB, K, x,
                                                       rule=si_hip.ARGMAX_FIRST_GREATER,
                                                       want_logits=False)
    assert first == top == O.argmax_first_greater(y32)
    return tok


def test_config4_head_argmax_full_vocab(hip_ctx, head):
    w, H = head
    _head_check(hip_ctx, w, H, si_hip.synth_normal(4002, K), "head 151936 x 5120")


def test_config4_chained_q5k_then_head(hip_ctx, head):
    """The head on the Q5_K matvec's GPU output (the chained path): the oracle
    evaluates the head on the same y5."""
    w, H = head
    w5 = si_hip.synth_matrix(Q5, seed=4201, rows=K, cols=K, threads=8)
    W5 = hip_ctx.upload_quant_weight_private(w5, Q5)
    x = si_hip.synth_normal(4202, K)
    y5 = hip_ctx.gguf_quant_matvec_weight(W5, K, K, x)
    _, y64, ab = O.matvec(Q5, w5, K, K, x, threads=8)
    assert_dot_close(y5, y64, ab, what="Q5_K before the head")
    _head_check(hip_ctx, w, H, y5, "chained Q5_K -> head")


def test_config4_embedding_full_table(hip_ctx):
    table = si_hip.synth_matrix(Q4, seed=4301, rows=VOCAB, cols=K, threads=16)
    T = hip_ctx.upload_quant_weight_private(table, Q4)
    try:
        ids = si_hip.synth_token_ids(4302, 64, VOCAB)
        ids[0], ids[1] = 0, VOCAB - 1
        got = hip_ctx.q4_k_embedding_tokens(T, (K, VOCAB), ids)
        rb = K // 256 * 144
        for i, t in enumerate(ids):
            exp = O.dequantize(Q4, table[int(t) * rb:(int(t) + 1) * rb], K)
            assert np.array_equal(got[i].view(np.uint32), exp.view(np.uint32)), f"id {t}"
    finally:
        T.free()


@pytest.mark.parametrize("batch", [2, 4, 8, 16])
def test_config5_matmul_many_full_size(hip_ctx, batch):
    log(f"config 5: M = {batch} on 17408 x 5120")
    w = si_hip.synth_matrix(Q4, seed=5001, rows=N, cols=K, threads=16)
    X = si_hip.synth_normal(5002 + batch, batch * K).reshape(batch, K)
    W = hip_ctx.upload_quant_weight_private(w, Q4)
    outs = hip_ctx.gguf_quant_matmul_many_weight(W, N, K, batch, X)
    for b in range(batch):
        _, y64, ab = O.matvec(Q4, w, N, K, X[b], threads=16)
        assert_dot_close(outs[b], y64, ab, what=f"M={batch} candidate {b}")
    W.free()


# ---- config 5b: the 64-layer aggregate's per-layer shapes ---------------------------------
# bench.py streams 64 synthetic 27B-class layers per token: Q4_K 16384 x 5120
# (q/k/v), Q4_K 5120 x 6144 (o), the fused Q4_K gate/up 17408 x 5120 and the
# Q6_K down 5120 x 17408 (the reference's layer loop, qwen35_runtime.rs:1809-1938).
@pytest.mark.parametrize("rows,cols", [(16384, 5120), (5120, 6144)])
def test_config5_aggregate_layer_shapes(hip_ctx, rows, cols):
    log(f"config 5 aggregate layer shape Q4_K {rows} x {cols}")
    w = si_hip.synth_matrix(Q4, seed=6000 + rows, rows=rows, cols=cols, threads=16)
    x = si_hip.synth_normal(6001 + cols, cols)
    _, y64, ab = O.matvec(Q4, w, rows, cols, x, threads=16)
    W = hip_ctx.upload_quant_weight_private(w, Q4)
    try:
        y = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
    finally:
        W.free()
    worst = assert_dot_close(y, y64, ab, what=f"layer {rows}x{cols}")
    log(f"  worst {worst:.4f} of the bar")


def test_config5_aggregate_token_matches_single_calls(hip_ctx):
    """Two layers of the aggregate's token, issued as bench.py issues them (the
    device-resident calls back to back on the context's stream, one wait at
    the end), give the same bits as the synchronous host calls one by one."""
    import ctypes as C
    lib = si_hip.lib()
    shapes = [(Q4, 16384, 5120), (Q4, 5120, 6144), (Q4, N, K), (Q4, N, K), (Q6, K, N)]
    layers = []
    for layer in range(2):
        layers.append([hip_ctx.upload_quant_weight_private(
            si_hip.synth_matrix(t, seed=6100 + 10 * layer + i, rows=r, cols=c, threads=16), t)
            for i, (t, r, c) in enumerate(shapes)])
    x6 = si_hip.synth_normal(6200, 6144)
    xk = x6[:K].copy()
    xm = (si_hip.synth_normal(6201, K) * np.float32(0.1)).astype(np.float32)
    d_x6, d_xk, d_xm = (hip_ctx.device_alloc(a.nbytes) for a in (x6, xk, xm))
    for p, a in ((d_x6, x6), (d_xk, xk), (d_xm, xm)):
        hip_ctx.to_device(p, a)
    outs = [(hip_ctx.device_alloc(16384 * 4), hip_ctx.device_alloc(K * 4),
             hip_ctx.device_alloc(N * 4), hip_ctx.device_alloc(K * 4)) for _ in layers]
    try:
        for L, (yq, yo, h, yd) in zip(layers, outs):
            si_hip._check(lib.si_hip_quant_matvec_device(hip_ctx.handle, L[0].handle, 16384, K,
                                                         C.c_void_p(d_xk), C.c_void_p(yq)))
            si_hip._check(lib.si_hip_quant_matvec_device(hip_ctx.handle, L[1].handle, K, 6144,
                                                         C.c_void_p(d_x6), C.c_void_p(yo)))
            si_hip._check(lib.si_hip_fused_mlp_device(hip_ctx.handle, L[2].handle, L[3].handle,
                                                      L[4].handle, N, K, K, C.c_void_p(d_xm),
                                                      C.c_void_p(h), C.c_void_p(yd)))
        hip_ctx.synchronize()
        for i, (L, (yq, yo, h, yd)) in enumerate(zip(layers, outs)):
            log(f"  layer {i}: device token against single host calls")
            assert np.array_equal(hip_ctx.from_device(yq, (16384,)),
                                  hip_ctx.gguf_quant_matvec_weight(L[0], 16384, K, xk))
            assert np.array_equal(hip_ctx.from_device(yo, (K,)),
                                  hip_ctx.gguf_quant_matvec_weight(L[1], K, 6144, x6))
            assert np.array_equal(hip_ctx.from_device(yd, (K,)),
                                  hip_ctx.gguf_quant_fused_mlp_weights(L[2], L[3], L[4], N, K, K,
                                                                       xm))
    finally:
        for L in layers:
            for w in L:
                w.free()
        for p in (d_x6, d_xk, d_xm):
            hip_ctx.device_free(p)
        for group in outs:
            for p in group:
                hip_ctx.device_free(p)
