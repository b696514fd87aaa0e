"""GPU: residency of borrowed weight bytes in HBM.

The reference's byte-slice entry points bind the caller's host bytes to the
GPU without a copy (unified memory); here a context keeps an HBM copy of each
borrowed range, keyed by (host address, length), under a byte budget.  These
tests read the context's residency counters: the second call on the same
bytes copies nothing, a change inside a sampled window or an eviction copies
again, a budget of 0 or below the call's bytes stages per call, and the GGUF
store's row ranges of one tensor share one resident copy.  Results are the
same bits whichever way the bytes reached HBM.
"""
import numpy as np
import pytest

import oracle_lib as O
import si_hip
from test_gpu_parity import assert_dot_close, same_bits
from test_gguf import GgufFile, _kquant_file

pytestmark = pytest.mark.gpu

Q4, Q5, Q6 = 12, 13, 14


@pytest.fixture
def rctx(hip_ctx):
    hip_ctx.set_residency_budget(si_hip.DEFAULT_RESIDENCY_BUDGET)
    hip_ctx.residency_evict()
    yield hip_ctx
    hip_ctx.set_residency_budget(si_hip.DEFAULT_RESIDENCY_BUDGET)
    hip_ctx.residency_evict()


def _delta(a, b):
    return {k: b[k] - a[k] for k in ("hits", "uploads", "uploaded_bytes", "evictions")}


def test_second_call_copies_no_weights(rctx):
    rows, cols = 4096, 5120
    w = si_hip.synth_matrix(Q4, seed=8100, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(8101, cols)
    s0 = rctx.residency_stats()
    y1 = rctx.q4_k_matvec(w, rows, cols, x)
    s1 = rctx.residency_stats()
    assert _delta(s0, s1) == {"hits": 0, "uploads": 1, "uploaded_bytes": w.size, "evictions": 0}
    assert s1["resident_ranges"] == 1 and s1["resident_bytes"] == w.size
    y2 = rctx.q4_k_matvec(w, rows, cols, x)
    s2 = rctx.residency_stats()
    assert _delta(s1, s2) == {"hits": 1, "uploads": 0, "uploaded_bytes": 0, "evictions": 0}
    assert same_bits(y1, y2)
    _, y64, ab = O.matvec(Q4, w, rows, cols, x, threads=8)
    assert_dot_close(y2, y64, ab, what="resident weights")
    # the same bytes through the generic entry point share the range
    y3 = rctx.gguf_quant_matvec_bytes(Q4, w, rows, cols, x)
    assert _delta(s2, rctx.residency_stats())["hits"] == 1
    assert same_bits(y1, y3)


def test_changed_bytes_are_copied_again(rctx):
    rows, cols = 512, 2048
    w = si_hip.synth_matrix(Q4, seed=8200, rows=rows, cols=cols)
    x = si_hip.synth_normal(8201, cols)
    y1 = rctx.q4_k_matvec(w, rows, cols, x)
    # block 0 of row 0 lies in the first sampled window: scale its d by 2
    d = np.frombuffer(w[0:2].tobytes(), np.float16)[0]
    w[0:2] = np.frombuffer(np.float16(d * 2).tobytes(), np.uint8)
    s0 = rctx.residency_stats()
    y2 = rctx.q4_k_matvec(w, rows, cols, x)
    s1 = rctx.residency_stats()
    assert _delta(s0, s1)["uploads"] == 1 and _delta(s0, s1)["hits"] == 0
    _, y64, ab = O.matvec(Q4, w, rows, cols, x)
    assert_dot_close(y2, y64, ab, what="changed bytes")
    assert y2[0] != y1[0] and same_bits(y2[1:], y1[1:])
    # an eviction of an overlapping range forces the next copy
    rctx.residency_evict(w[100:200])
    s2 = rctx.residency_stats()
    assert s2["resident_ranges"] == 0 and _delta(s1, s2)["evictions"] == 1
    y3 = rctx.q4_k_matvec(w, rows, cols, x)
    assert _delta(s2, rctx.residency_stats())["uploads"] == 1
    assert same_bits(y2, y3)


def _unsampled_byte(nbytes, lo):
    """An offset at or past `lo` that none of the resident-range fingerprint's
    64 windows of 64 bytes covers (windows at (len - 64) // 63 * k)."""
    step = (nbytes - 64) // 63
    for off in range(lo, nbytes):
        k = off // step
        if not any(o <= off < o + 64 for o in (step * k, step * (k + 1)) if o <= nbytes - 64):
            return off
    raise AssertionError("every byte sampled")


def test_change_outside_the_sampled_windows_needs_evict(rctx):
    """The documented contract (si_hip.h, residency): bytes changed in place
    outside the sampled windows go unseen, so the next call reuses the
    resident copy, bit for bit; si_hip_residency_evict on the changed range
    makes the next call copy the new bytes."""
    rows, cols = 512, 2048
    w = si_hip.synth_matrix(Q4, seed=8250, rows=rows, cols=cols)
    x = si_hip.synth_normal(8251, cols)
    y1 = rctx.q4_k_matvec(w, rows, cols, x)
    rb = w.size // rows
    # a qs byte of some row, between two windows: its low nibble's weight moves
    off = _unsampled_byte(w.size, 100 * rb + 40)
    assert (off % 144) >= 16  # a qs byte, not a block header
    row = off // rb
    w[off] ^= 0x0F
    s0 = rctx.residency_stats()
    y2 = rctx.q4_k_matvec(w, rows, cols, x)
    assert _delta(s0, rctx.residency_stats()) == {"hits": 1, "uploads": 0, "uploaded_bytes": 0,
                                                  "evictions": 0}
    assert same_bits(y2, y1)  # the stale resident copy, as documented
    rctx.residency_evict(w[off:off + 1])
    s1 = rctx.residency_stats()
    y3 = rctx.q4_k_matvec(w, rows, cols, x)
    assert _delta(s1, rctx.residency_stats())["uploads"] == 1
    _, y64, ab = O.matvec(Q4, w, rows, cols, x)
    assert_dot_close(y3, y64, ab, what="after the evict")
    assert y3[row] != y1[row]


def test_budget_zero_and_small_budget_stage_per_call(rctx):
    rows, cols = 1024, 1024
    w = si_hip.synth_matrix(Q6, seed=8300, rows=rows, cols=cols)
    x = si_hip.synth_normal(8301, cols)
    ref = rctx.q6_k_matvec(w, rows, cols, x)
    for budget in (0, w.size - 1):
        rctx.set_residency_budget(budget)
        s0 = rctx.residency_stats()
        assert s0["resident_ranges"] == 0  # shrinking the budget evicted the range
        for _ in range(2):
            assert same_bits(rctx.q6_k_matvec(w, rows, cols, x), ref)
        s1 = rctx.residency_stats()
        assert _delta(s0, s1)["uploads"] == 2 and _delta(s0, s1)["hits"] == 0
        assert s1["resident_ranges"] == 0
    # a budget for two matrices of three: the least recently used one goes
    rctx.set_residency_budget(2 * w.size)
    ws = [si_hip.synth_matrix(Q6, seed=8310 + i, rows=rows, cols=cols) for i in range(3)]
    for m in ws:
        rctx.q6_k_matvec(m, rows, cols, x)
    s = rctx.residency_stats()
    assert s["resident_ranges"] == 2 and s["resident_bytes"] == 2 * w.size
    before = rctx.residency_stats()
    rctx.q6_k_matvec(ws[2], rows, cols, x)  # most recent: still resident
    rctx.q6_k_matvec(ws[0], rows, cols, x)  # evicted: copied again
    d = _delta(before, rctx.residency_stats())
    assert d["hits"] == 1 and d["uploads"] == 1 and d["evictions"] == 1


def test_fused_gate_up_group_and_matmul_bytes_are_resident(rctx):
    rows, cols = 768, 2048
    g = si_hip.synth_matrix(Q4, seed=8400, rows=rows, cols=cols)
    u = si_hip.synth_matrix(Q4, seed=8401, rows=rows, cols=cols)
    x = si_hip.synth_normal(8402, cols)
    h1 = rctx.q4_k_fused_gate_up(g, u, rows, cols, x)
    s0 = rctx.residency_stats()
    h2 = rctx.q4_k_fused_gate_up(g, u, rows, cols, x)
    assert _delta(s0, rctx.residency_stats())["hits"] == 2
    assert same_bits(h1, h2)
    G = rctx.upload_quant_weight_private(g, Q4)
    U = rctx.upload_quant_weight_private(u, Q4)
    assert same_bits(rctx.q4_k_fused_gate_up_weights(G, U, rows, cols, x), h1)
    G.free(); U.free()
    # grouped bytes: both matrices already resident
    s1 = rctx.residency_stats()
    outs = rctx.gguf_quant_matvec_many_bytes([(Q4, g, rows, cols), (Q4, u, rows, cols)], x)
    d = _delta(s1, rctx.residency_stats())
    assert d["hits"] == 2 and d["uploads"] == 0
    _, y64, ab = O.matvec(Q4, g, rows, cols, x)
    assert_dot_close(outs[0], y64, ab, what="grouped bytes")
    X = si_hip.synth_normal(8403, 3 * cols).reshape(3, cols)
    s2 = rctx.residency_stats()
    m = rctx.gguf_quant_matmul_many_bytes(Q4, g, rows, cols, 3, X)
    assert _delta(s2, rctx.residency_stats())["hits"] == 1
    for b in range(3):
        _, y64, ab = O.matvec(Q4, g, rows, cols, X[b])
        assert_dot_close(m[b], y64, ab, what=f"matmul bytes {b}")


def test_store_row_ranges_share_one_resident_tensor(rctx):
    rows, cols, mats, data = _kquant_file(21)
    g = GgufFile(data=data)
    x = si_hip.synth_normal(22, cols)
    try:
        s0 = rctx.residency_stats()
        a = g.matvec_tensor_rows(rctx, "q4", 0, 40, x)
        b = g.matvec_tensor_rows(rctx, "q4", 40, rows - 40, x)
        c = g.matvec_tensor_rows(rctx, "q4", 0, rows, x)
        d = _delta(s0, rctx.residency_stats())
        assert d["uploads"] == 1 and d["hits"] == 2
        # (a row range may take another launch form than the whole tensor:
        # the same rows agree within the bound, not always to the bit)
        _, y64, ab = O.matvec(Q4, mats["q4"], rows, cols, x)
        assert_dot_close(c, y64, ab, what="store rows")
        assert_dot_close(np.concatenate([a, b]), y64, ab, what="store row ranges")
    finally:
        g.close()


def test_view_rows_match_store_and_share_residency(rctx):
    """gguf_quant_matvec_tensor_rows over a GgufTensorView (the payload bytes
    a caller holds): the same bits as the store's call on the same rows, and
    row ranges of one payload share one resident copy (ranges of other row
    counts within the bound)."""
    rows, cols, mats, data = _kquant_file(31)
    g = GgufFile(data=data)
    x = si_hip.synth_normal(32, cols)
    try:
        for name, t in (("q4", Q4), ("q5", Q5), ("q6", Q6)):
            payload = np.ascontiguousarray(mats[name])
            s0 = rctx.residency_stats()
            a = rctx.gguf_quant_matvec_view_rows(name, t, (cols, rows), payload, 3, 50, x)
            b = rctx.gguf_quant_matvec_view_rows(name, t, (cols, rows), payload, 53, rows - 53, x)
            d = _delta(s0, rctx.residency_stats())
            assert d["uploads"] == 1 and d["hits"] == 1
            whole = g.matvec_tensor_rows(rctx, name, 0, rows, x)
            _, y64, ab = O.matvec(t, mats[name], rows, cols, x)
            assert_dot_close(np.concatenate([a, b]), y64[3:], ab[3:], what=f"{name} view rows")
            assert same_bits(g.matvec_tensor_rows(rctx, name, 3, 50, x), a)
            assert_dot_close(whole, y64, ab, what=f"{name} store rows")
    finally:
        g.close()


def test_embedding_view_is_bit_exact_and_resident(rctx):
    rows, cols = 512, 1024
    table = si_hip.synth_matrix(Q4, seed=8500, rows=rows, cols=cols)
    rb = cols // 256 * 144
    s0 = rctx.residency_stats()
    for tok in (0, 17, rows - 1):
        got = rctx.q4_k_embedding_view(Q4, (cols, rows), table, tok)
        exp = O.dequantize(Q4, table[tok * rb:(tok + 1) * rb], cols)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), tok
    d = _delta(s0, rctx.residency_stats())
    assert d["uploads"] == 1 and d["hits"] == 2  # the table went to HBM once
    # with residency off, the row alone is copied (same bits)
    rctx.set_residency_budget(0)
    got = rctx.q4_k_embedding_view(Q4, (cols, rows), table, 17)
    exp = O.dequantize(Q4, table[17 * rb:18 * rb], cols)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
