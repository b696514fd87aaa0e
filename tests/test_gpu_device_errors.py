"""GPU: the Q6_K output head with the argmax fused into its kernel, and the
failure reports of kernels that cannot finish their work correctly.

  * the fused head (the Q6_K matrix-core kernel stores the logits and keeps
    each workgroup's best candidate; the workgroups reduce theirs through the
    workspace) against the generic policy's separate argmax kernel and the
    oracle's two tie rules (src/runtime.rs:4301-4309, qwen35_runtime.rs:
    2237-2244), on crafted ties, non-finite logits and odd vocabularies;
  * an embedding token id beyond the table on the device path gives a NaN
    row and SI_HIP_ERR_DEVICE at the next synchronisation, and the context
    works normally afterwards;
  * the embedding checks in q4_k_embedding_tensor's order (src/metal.rs:
    3785-3810): a table shorter than its shape serves the rows it holds;
  * bounded waits driven to give up by the test hook (every kernel still
    ends): the split-tile and K-slice combines and the argmax reduction
    report, the call fails with SI_HIP_ERR_DEVICE, and the next calls are
    correct again.
"""
import ctypes as C
import struct

import numpy as np
import pytest

import oracle_lib as O
import si_hip
from test_gpu_parity import assert_dot_close, log, same_bits

pytestmark = pytest.mark.gpu

Q4, Q6 = 12, 14
P = C.c_void_p


def _q6_dominant_block():
    """A Q6_K block whose 256 weights are all 31 * 127 (d = 1, every scale
    127, every 6-bit quant 63)."""
    b = bytearray(210)
    b[0:128] = b"\xff" * 128       # ql
    b[128:192] = b"\xff" * 64      # qh
    b[192:208] = bytes([127]) * 16  # scales
    b[208:210] = struct.pack("<H", 0x3C00)
    return bytes(b)


@pytest.mark.parametrize("rows", [4096 + 5, 20011])
def test_fused_head_tie_rules(hip_ctx, rows):
    cols = 512
    w = si_hip.synth_matrix(Q6, seed=7100 + rows, rows=rows, cols=cols)
    blocks = w.reshape(rows, 2, 210).copy()
    dom = np.frombuffer(_q6_dominant_block(), np.uint8)
    for r in (17, rows // 2, rows - 1):
        blocks[r, :] = dom
    x = np.ones(cols, np.float32)
    H = hip_ctx.upload_quant_weight_private(blocks.tobytes(), Q6)
    try:
        last, logits = hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x)
        assert logits[17] == logits[rows // 2] == logits[rows - 1] == logits.max()
        first, _ = hip_ctx.gguf_quant_matvec_argmax_weight(
            H, rows, cols, x, rule=si_hip.ARGMAX_FIRST_GREATER, want_logits=False)
        assert (first, last) == (17, rows - 1)
        assert last == O.argmax_last_finite(logits)
        assert first == O.argmax_first_greater(logits)
        # the generic policy (matvec, then the separate argmax kernel) agrees
        hip_ctx.set_kernel_policy(si_hip.KERNEL_GENERIC)
        try:
            g_last, _ = hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x)
            g_first, _ = hip_ctx.gguf_quant_matvec_argmax_weight(
                H, rows, cols, x, rule=si_hip.ARGMAX_FIRST_GREATER)
        finally:
            hip_ctx.set_kernel_policy(si_hip.KERNEL_AUTO)
        assert (g_first, g_last) == (first, last)
    finally:
        H.free()


def test_fused_head_no_finite_logits(hip_ctx):
    """d = +inf with nonzero scales: every logit is +inf or NaN."""
    rows, cols = 40, 512
    b = bytearray(si_hip.synth_matrix(Q6, seed=7200, rows=rows, cols=cols).tobytes())
    for r in range(rows):
        for k in range(2):
            off = (2 * r + k) * 210
            b[off + 208:off + 210] = struct.pack("<H", 0x7C00)
            b[off + 192:off + 208] = bytes([5]) * 16
    H = hip_ctx.upload_quant_weight_private(bytes(b), Q6)
    x = si_hip.synth_normal(7201, cols)
    try:
        with pytest.raises(si_hip.HipError) as e:
            hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x)
        assert e.value.status == -8
        tok, logits = hip_ctx.gguf_quant_matvec_argmax_weight(
            H, rows, cols, x, rule=si_hip.ARGMAX_FIRST_GREATER)
        assert not np.any(np.isfinite(logits))
        assert tok == O.argmax_first_greater(logits)
    finally:
        H.free()


def test_fused_head_matches_separate_argmax_kernel(hip_ctx):
    """Random head 32000 x 5120: the fused kernel's logits equal the plain
    matvec's bit for bit, its token the separate argmax's, under both rules."""
    rows, cols = 32000, 5120
    w = si_hip.synth_matrix(Q6, seed=7300, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(7301, cols)
    H = hip_ctx.upload_quant_weight_private(w, Q6)
    try:
        y = hip_ctx.gguf_quant_matvec_weight(H, rows, cols, x)
        for rule, pick in ((si_hip.ARGMAX_LAST_FINITE, O.argmax_last_finite),
                           (si_hip.ARGMAX_FIRST_GREATER, O.argmax_first_greater)):
            tok, logits = hip_ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x, rule=rule)
            assert same_bits(logits, y)
            assert tok == pick(y)
        _, y64, ab = O.matvec(Q6, w, rows, cols, x, threads=8)
        assert_dot_close(y, y64, ab, what="head logits")
    finally:
        H.free()


def _embedding_device(hip_ctx, T, shape, ids):
    lib = si_hip.lib()
    cols = shape[0]
    ids = np.asarray(ids, np.uint32)
    d_ids = hip_ctx.device_alloc(ids.size * 4)
    d_out = hip_ctx.device_alloc(ids.size * cols * 4)
    try:
        hip_ctx.to_device(d_ids, ids)
        rc = lib.si_hip_embedding_device(hip_ctx.handle, T.handle, shape[0], shape[1], P(d_ids),
                                         ids.size, P(d_out))
        assert rc == 0, si_hip.last_error()
        err = None
        try:
            hip_ctx.synchronize()
        except si_hip.HipError as e:
            err = e
        out = hip_ctx.from_device(d_out, ids.size * cols).reshape(ids.size, cols)
        return out, err
    finally:
        hip_ctx.device_free(d_ids)
        hip_ctx.device_free(d_out)


def test_embedding_device_id_beyond_table_reports(hip_ctx):
    rows, cols = 64, 512
    table = si_hip.synth_matrix(Q4, seed=7400, rows=rows, cols=cols)
    T = hip_ctx.upload_quant_weight_private(table, Q4)
    rb = cols // 256 * 144
    try:
        out, err = _embedding_device(hip_ctx, T, (cols, rows), [3, rows, 5, 0xFFFFFFFF])
        assert err is not None and err.status == -9
        assert "token id" in err.message
        assert np.all(np.isnan(out[1])) and np.all(np.isnan(out[3]))
        for i, t in ((0, 3), (2, 5)):
            exp = O.dequantize(Q4, table[t * rb:(t + 1) * rb], cols)
            assert np.array_equal(out[i].view(np.uint32), exp.view(np.uint32))
        # the context is clean afterwards: device and host paths both work
        out2, err2 = _embedding_device(hip_ctx, T, (cols, rows), [rows - 1])
        assert err2 is None
        exp = O.dequantize(Q4, table[(rows - 1) * rb:rows * rb], cols)
        assert np.array_equal(out2[0].view(np.uint32), exp.view(np.uint32))
        W = si_hip.synth_matrix(Q4, seed=7401, rows=4096, cols=5120, threads=8)
        Wh = hip_ctx.upload_quant_weight_private(W, Q4)
        xv = si_hip.synth_normal(7402, 5120)
        _, y64, ab = O.matvec(Q4, W, 4096, 5120, xv, threads=8)
        assert_dot_close(hip_ctx.gguf_quant_matvec_weight(Wh, 4096, 5120, xv), y64, ab,
                         what="after the report")
        Wh.free()
    finally:
        T.free()


def test_embedding_truncated_table_serves_rows_it_holds(hip_ctx):
    """A table uploaded with fewer bytes than its shape (rows 0..9 of 16)
    serves those rows; row 12 fails on the payload check (the reference's
    order: type, id and dimension, offsets, then that row's bytes), and on
    the device path gives a NaN row and a report."""
    rows, cols = 16, 256
    held = 10
    table = si_hip.synth_matrix(Q4, seed=7500, rows=rows, cols=cols)
    T = hip_ctx.upload_quant_weight_private(table[:held * 144], Q4)
    try:
        got = hip_ctx.q4_k_embedding_tensor(T, (cols, rows), held - 1)
        exp = O.dequantize(Q4, table[(held - 1) * 144:held * 144], cols)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
        with pytest.raises(si_hip.HipError) as e:
            hip_ctx.q4_k_embedding_tensor(T, (cols, rows), 12)
        assert e.value.status == -3
        assert e.value.message == "Q4_K embedding tensor payload is shorter than its shape"
        with pytest.raises(si_hip.HipError) as e:
            hip_ctx.q4_k_embedding_tensor(T, (cols, rows), rows)
        assert e.value.message == "Q4_K embedding token id or dimension is invalid"
        with pytest.raises(si_hip.HipError) as e:
            hip_ctx.q4_k_embedding_tensor(T, (cols + 1, rows), 0)
        assert e.value.message == "Q4_K embedding token id or dimension is invalid"
        with pytest.raises(si_hip.HipError) as e:
            hip_ctx.q4_k_embedding_tensor(T, (0, rows), 0)
        assert e.value.message == "Q4_K embedding dimension is invalid"
        out, err = _embedding_device(hip_ctx, T, (cols, rows), [2, 12])
        assert err is not None and err.status == -9
        assert np.all(np.isnan(out[1]))
        exp = O.dequantize(Q4, table[2 * 144:3 * 144], cols)
        assert np.array_equal(out[0].view(np.uint32), exp.view(np.uint32))
    finally:
        T.free()


@pytest.fixture
def give_up(hip_ctx):
    hip_ctx.debug_set_wait_give_up(16)
    yield hip_ctx
    hip_ctx.debug_set_wait_give_up(0)


def test_forced_give_up_in_split_combine_reports(give_up):
    """17408 x 5120 Q4_K runs as a split launch: with the hook set, every
    combine of a split tile gives up after 16 polls and reports."""
    ctx = give_up
    rows, cols = 17408, 5120
    w = si_hip.synth_matrix(Q4, seed=7600, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(7601, cols)
    W = ctx.upload_quant_weight_private(w, Q4)
    try:
        log("forced give-up: split combine")
        with pytest.raises(si_hip.HipError) as e:
            ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        assert e.value.status == -9 and "split tile" in e.value.message
        ctx.debug_set_wait_give_up(0)
        _, y64, ab = O.matvec(Q4, w, rows, cols, x, threads=8)
        assert_dot_close(ctx.gguf_quant_matvec_weight(W, rows, cols, x), y64, ab,
                         what="after the forced give-up")
    finally:
        W.free()


def test_forced_give_up_in_sliced_combine_reports(give_up):
    """2560 x 17408 Q6_K (a down projection) runs K-sliced: with the hook set,
    the wave that completes a tile's count gives up waiting for the other
    slices' sums after 16 polls and reports; with it cleared, the same call
    is within its bound again (the entries and counters were restored)."""
    ctx = give_up
    rows, cols = 2560, 17408
    w = si_hip.synth_matrix(Q6, seed=7650, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(7651, cols)
    W = ctx.upload_quant_weight_private(w, Q6)
    try:
        log("forced give-up: sliced combine")
        with pytest.raises(si_hip.HipError) as e:
            ctx.gguf_quant_matvec_weight(W, rows, cols, x)
        assert e.value.status == -9 and "split tile" in e.value.message
        ctx.debug_set_wait_give_up(0)
        _, y64, ab = O.matvec(Q6, w, rows, cols, x, threads=8)
        assert_dot_close(ctx.gguf_quant_matvec_weight(W, rows, cols, x), y64, ab,
                         what="after the forced give-up")
    finally:
        W.free()


@pytest.mark.parametrize("policy", [si_hip.KERNEL_AUTO, si_hip.KERNEL_GENERIC],
                         ids=["fused", "separate"])
def test_forced_give_up_in_argmax_reports(give_up, policy):
    ctx = give_up
    rows, cols = 4096, 1024
    w = si_hip.synth_matrix(Q6, seed=7700, rows=rows, cols=cols)
    x = si_hip.synth_normal(7701, cols)
    H = ctx.upload_quant_weight_private(w, Q6)
    ctx.set_kernel_policy(policy)
    try:
        log(f"forced give-up: argmax, policy {policy}")
        with pytest.raises(si_hip.HipError) as e:
            ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x)
        assert e.value.status == -9 and "argmax" in e.value.message
        ctx.debug_set_wait_give_up(0)
        tok, logits = ctx.gguf_quant_matvec_argmax_weight(H, rows, cols, x)
        assert tok == O.argmax_last_finite(logits)
    finally:
        ctx.set_kernel_policy(si_hip.KERNEL_AUTO)
        H.free()
