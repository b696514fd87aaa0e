"""GPU: outputs of the synchronous host calls.

A synchronous call's last kernel stores its output straight into the
context's pinned staging when it takes at most 16 MB there; larger outputs
land in device staging and are copied to the caller's buffer.  These tests
take both branches, one after the other on one context: a whole-tensor
dequantize and a batch of embedding rows above 16 MB, the same calls below
it, and a matvec between them, each bit-exact against the oracle (the
dequantize and embedding rows) or within its bound (the matvec).
"""
import sys

import numpy as np
import pytest

import oracle_lib as O
import si_hip
from test_gpu_parity import assert_dot_close, same_bits

pytestmark = pytest.mark.gpu

Q4, Q6 = 12, 14


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_dequantize_above_and_below_the_pinned_limit(hip_ctx):
    big, small = 20000, 3000  # 20.5 MB and 3.1 MB of f32 output
    data = si_hip.synth_blocks(Q6, seed=5100, n_blocks=big)
    exp = O.dequantize(Q6, data, big * 256)
    rb = si_hip.BLOCK_BYTES[Q6]
    for rep in range(2):
        log(f"dequantize {big} blocks, rep {rep}")
        assert same_bits(hip_ctx.dequantize(Q6, data, big * 256), exp)
        log(f"dequantize {small} blocks, rep {rep}")
        assert same_bits(hip_ctx.dequantize(Q6, data[:small * rb], small * 256),
                         exp[:small * 256])


def test_embedding_rows_above_the_pinned_limit(hip_ctx):
    vocab, cols = 2048, 5120
    table = si_hip.synth_matrix(Q4, seed=5200, rows=vocab, cols=cols, threads=8)
    T = hip_ctx.upload_quant_weight_private(table, Q4)
    rb = cols // 256 * 144
    try:
        for n in (1100, 64, 1100):  # 22.5 MB, 1.3 MB, 22.5 MB of rows
            log(f"embedding {n} ids")
            ids = si_hip.synth_token_ids(5201 + n, n, vocab)
            got = hip_ctx.q4_k_embedding_tokens(T, (cols, vocab), ids)
            for i in (0, n // 2, n - 1):
                t = int(ids[i])
                assert same_bits(got[i], O.dequantize(Q4, table[t * rb:(t + 1) * rb], cols))
            # every row: the table's rows at the ids, dequantized once
            rows = O.dequantize(Q4, table, vocab * cols).reshape(vocab, cols)
            assert same_bits(got, rows[ids])
    finally:
        T.free()


def test_matvec_between_large_host_outputs(hip_ctx):
    rows, cols = 17408, 5120
    w = si_hip.synth_matrix(Q4, seed=5300, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(5301, cols)
    _, y64, ab = O.matvec(Q4, w, rows, cols, x, threads=8)
    W = hip_ctx.upload_quant_weight_private(w, Q4)
    data = si_hip.synth_blocks(Q4, seed=5302, n_blocks=17000)  # 17.4 MB of output
    exp = O.dequantize(Q4, data, 17000 * 256)
    try:
        y0 = hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        assert_dot_close(y0, y64, ab, what="first matvec")
        assert same_bits(hip_ctx.dequantize(Q4, data, 17000 * 256), exp)
        assert same_bits(hip_ctx.gguf_quant_matvec_weight(W, rows, cols, x), y0)
    finally:
        W.free()
