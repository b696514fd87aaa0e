"""GPU: si_hip_quant_matvec_noalloc (the matvec that allocates nothing)
against si_hip_quant_matvec_device, through the C ABI.

The two run the same kernels; the no-alloc one combines split tiles and K
slices in its static device workspace instead of a context's.  Results must be bit-identical
(the combine order is fixed for a given grid), and therefore within the
oracle's 2e-5 * sum|w*x| bar.  Each type runs two calls in a row, the second
on a smaller matrix, so the second finds the workspace as the first left it.

A kernel that gives up a bounded wait records it in the library's device
failure word; si_hip_noalloc_check reports it (SI_HIP_ERR_DEVICE), clears it
and puts the workspace back into its rest state.  The give-up is forced from
the host with the test hook (every wait gives up after 16 polls), so every
kernel still ends normally.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
import si_hip

pytestmark = pytest.mark.gpu

CASES = [  # (type, (rows, cols) of the first call, (rows, cols) of the second)
    (12, (17408, 5120), (1024, 5120)),
    (13, (5120, 5120), (300, 2304)),
    (14, (20011, 5120), (5120, 17408)),
    # K-sliced launches (the slices' sums meet in the workspace's entries)
    (12, (5120, 17408), (640, 17408)),
    (14, (2560, 17408), (16, 12288)),
]


def _hip():
    return C.CDLL("libamdhip64.so")


def _noalloc(w, t, rows, cols, d_x, d_y):
    return si_hip.lib().si_hip_quant_matvec_noalloc(
        t, C.c_void_p(w.device_ptr()), w.byte_len(), rows, cols, C.c_void_p(d_x),
        C.c_void_p(d_y), None)


@pytest.mark.parametrize("t,first,second", CASES)
def test_noalloc_matches_device_entry_point(hip_ctx, t, first, second):
    hip = _hip()
    for rows, cols in (first, second):
        print(f"no-alloc matvec t={t} {rows}x{cols}", flush=True)
        w = si_hip.synth_matrix(t, seed=rows + cols + t, rows=rows, cols=cols, threads=8)
        x = si_hip.synth_normal(rows ^ cols, cols)
        W = hip_ctx.upload_quant_weight_private(w, t)
        d_x = hip_ctx.device_alloc(cols * 4)
        d_y = hip_ctx.device_alloc(rows * 4)
        d_ref = hip_ctx.device_alloc(rows * 4)
        try:
            hip_ctx.to_device(d_x, x)
            hip_ctx.synchronize()
            rc = _noalloc(W, t, rows, cols, d_x, d_y)
            assert rc == 0, si_hip.last_error()
            assert hip.hipDeviceSynchronize() == 0
            lib = si_hip.lib()
            rc = lib.si_hip_quant_matvec_device(hip_ctx.handle, W.handle, rows, cols,
                                                C.c_void_p(d_x), C.c_void_p(d_ref))
            assert rc == 0, si_hip.last_error()
            hip_ctx.synchronize()
            y = hip_ctx.from_device(d_y, (rows,))
            ref = hip_ctx.from_device(d_ref, (rows,))
        finally:
            for p in (d_x, d_y, d_ref):
                hip_ctx.device_free(p)
            W.free()
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
        _, y64, ab = O.matvec(t, w, rows, cols, x, threads=8)
        assert np.all(np.abs(y.astype(np.float64) - y64) <= 2e-5 * ab + 1e-30)


def test_noalloc_rejections(hip_ctx):
    lib = si_hip.lib()
    W = hip_ctx.upload_quant_weight_private(
        si_hip.synth_matrix(12, seed=1, rows=16, cols=256), 12)
    d = hip_ctx.device_alloc(1024)
    try:
        ptr, n = C.c_void_p(W.device_ptr()), W.byte_len()
        cases = [
            ((11, ptr, n, 16, 256), -5),
            ((12, ptr, n, 16, 255), -2),
            ((12, ptr, n + 1, 16, 256), -3),
            ((12, ptr, n, 4194048 + 16, 256), -2),
            ((12, None, n, 16, 256), -1),
        ]
        for (t, p, nb, rows, cols), status in cases:
            rc = lib.si_hip_quant_matvec_noalloc(t, p, nb, rows, cols, C.c_void_p(d),
                                                 C.c_void_p(d), None)
            assert rc == status, (t, rows, cols, rc, si_hip.last_error())
            assert si_hip.last_error()
    finally:
        hip_ctx.device_free(d)
        W.free()


# split-tile (17408 x 5120 Q4_K) and K-sliced (2560 x 17408 Q6_K) launches: the
# two kinds of bounded wait in the no-alloc path
@pytest.mark.parametrize("t,rows,cols", [(12, 17408, 5120), (14, 2560, 17408)])
def test_noalloc_give_up_is_reported(hip_ctx, t, rows, cols):
    hip = _hip()
    lib = si_hip.lib()
    w = si_hip.synth_matrix(t, seed=7700 + t, rows=rows, cols=cols, threads=8)
    x = si_hip.synth_normal(7701, cols)
    W = hip_ctx.upload_quant_weight_private(w, t)
    d_x = hip_ctx.device_alloc(cols * 4)
    d_y = hip_ctx.device_alloc(rows * 4)
    d_ref = hip_ctx.device_alloc(rows * 4)
    try:
        hip_ctx.to_device(d_x, x)
        hip_ctx.synchronize()
        assert lib.si_hip_noalloc_check(None) == 0, si_hip.last_error()
        print(f"no-alloc forced give-up t={t} {rows}x{cols}", flush=True)
        assert lib.si_hip_noalloc_debug_set_wait_give_up(16, None) == 0, si_hip.last_error()
        try:
            assert _noalloc(W, t, rows, cols, d_x, d_y) == 0, si_hip.last_error()
            rc = lib.si_hip_noalloc_check(None)
            assert rc == -9 and "gave up" in si_hip.last_error()
            assert lib.si_hip_noalloc_check(None) == 0  # the word was cleared
        finally:
            assert lib.si_hip_noalloc_debug_set_wait_give_up(0, None) == 0, si_hip.last_error()
        print(f"no-alloc after the give-up t={t} {rows}x{cols}", flush=True)
        assert _noalloc(W, t, rows, cols, d_x, d_y) == 0, si_hip.last_error()
        assert lib.si_hip_noalloc_check(None) == 0, si_hip.last_error()
        assert hip.hipDeviceSynchronize() == 0
        rc = lib.si_hip_quant_matvec_device(hip_ctx.handle, W.handle, rows, cols,
                                            C.c_void_p(d_x), C.c_void_p(d_ref))
        assert rc == 0, si_hip.last_error()
        hip_ctx.synchronize()
        y = hip_ctx.from_device(d_y, (rows,))
        ref = hip_ctx.from_device(d_ref, (rows,))
    finally:
        for p in (d_x, d_y, d_ref):
            hip_ctx.device_free(p)
        W.free()
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
