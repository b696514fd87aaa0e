"""F32 matvec and RMSNorm (include/si_hip_f32.h, the GGUF F32 entry points of
include/si_hip_gguf.h): the CPU oracle (oracle/f32_ref.c) pinned by closed
forms and invariants, host-side validation with the reference's messages
(src/metal.rs:2641-3110, 4780-4870; src/qwen35.rs:14-87), and on the GPU the
HIP kernels against the oracle and an f64 recomputation."""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np
import pytest

import oracle_lib as O
import si_hip
from si_hip import GgufFile, HipError

from test_gguf import write_gguf

RMS_TOL = 4e-6   # relative, per element: a few f32 roundings of the norm chain
DOT_TOL = 2e-5   # relative to sum |w * x|


def f64_rms(mode, x, w, heads, head_dim, eps, gate=None):
    x = np.asarray(x, np.float64).reshape(heads, head_dim)
    w = np.asarray(w, np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(axis=1, keepdims=True) + np.float64(np.float32(eps)))
    y = x * inv
    if mode == 0:
        y = y * w
    elif mode == 1:
        y = y * (1.0 + w)
    else:
        g = np.asarray(gate, np.float64).reshape(heads, head_dim)
        y = y * w * (g / (1.0 + np.exp(-g)))
    return y.reshape(-1)


def assert_rms_close(y, ref64, what=""):
    err = np.abs(y.astype(np.float64) - ref64)
    bound = RMS_TOL * np.abs(ref64) + 1e-30
    worst = float(np.max(err / bound))
    assert worst <= 1.0, f"{what}: worst {worst:.3f}x of {RMS_TOL} relative"


# ---- the oracle ----------------------------------------------------------------

def test_oracle_f32_matvec_reference_case_and_integers():
    # the reference's test matrix (src/metal.rs:7339-7345): exact small values
    w = np.array([1.0, 0.5, -1.0, 2.0, -2.0, 1.0, 0.25, 3.0, 0.125, -0.5, 2.0, -1.0], np.float32)
    x = np.array([2.0, -1.0, 0.5, 3.0], np.float32)
    assert O.f32_matvec(w, x, 3, 4).tolist() == [7.0, 4.125, -1.25]
    # integer-valued inputs stay exact in f32: the sequential sums are the integer dots
    rng = np.random.default_rng(3)
    wi = rng.integers(-50, 50, (17, 33))
    xi = rng.integers(-50, 50, 33)
    got = O.f32_matvec(wi.astype(np.float32), xi.astype(np.float32), 17, 33)
    assert np.array_equal(got.astype(np.int64), wi @ xi)


def test_oracle_rms_norm_closed_forms():
    # x = 2 everywhere: mean square 4, inverse exactly 1/2 when eps is negligible
    w = np.array([1.0, -3.0, 0.25, 7.0], np.float32)
    assert np.array_equal(O.rms_norm(0, [2, 2, 2, 2], w, 1, 4, 1e-30), w)
    assert np.array_equal(O.rms_norm(1, [2, -2, 2, -2], [0, 1, 3, -1], 1, 4, 1e-30),
                          np.array([1.0, -2.0, 4.0, -0.0], np.float32))
    # mean square 1/4 + eps 3/4 = 1: inverse exactly 1
    y = O.rms_norm(0, [0.5, -0.5], [3.0, 5.0], 1, 2, 0.75)
    assert y.tolist() == [1.5, -2.5]
    # the reference's test vector (src/metal.rs:7255-7266) against f64 arithmetic
    x, w = [1.0, -2.0, 3.0, -4.0], [1.0, 0.5, 2.0, -1.0]
    assert_rms_close(O.rms_norm(0, x, w, 1, 4, 1e-5), f64_rms(0, x, w, 1, 4, 1e-5), "mode 0")


def test_oracle_rms_norm_invariants():
    rng = np.random.default_rng(9)
    heads, hd = 6, 40
    x = rng.standard_normal(heads * hd).astype(np.float32)
    w = rng.standard_normal(hd).astype(np.float32)
    g = (rng.standard_normal(heads * hd) * 4).astype(np.float32)
    for mode in (1, 2):
        whole = O.rms_norm(mode, x, w, heads, hd, 1e-6, gate=g if mode == 2 else None)
        for h in range(heads):
            sl = slice(h * hd, (h + 1) * hd)
            one = O.rms_norm(mode, x[sl], w, 1, hd, 1e-6, gate=g[sl] if mode == 2 else None)
            assert np.array_equal(one, whole[sl])
        assert_rms_close(whole, f64_rms(mode, x, w, heads, hd, 1e-6, g), f"mode {mode}")
    # a power-of-two scale of x, with eps scaled by its square, changes no bit
    a = O.rms_norm(1, x, w, heads, hd, 2.0 ** -20)
    b = O.rms_norm(1, x * np.float32(8), w, heads, hd, 2.0 ** -14)
    assert np.array_equal(a, b)
    # silu(0) = 0: a zero gate zeroes the output; a large gate is the identity
    z = O.rms_norm(2, x[:hd], w, 1, hd, 1e-6, gate=np.zeros(hd, np.float32))
    assert np.all(z == 0.0)
    big = O.rms_norm(2, x[:hd], w, 1, hd, 1e-6, gate=np.full(hd, 40.0, np.float32))
    assert np.array_equal(big, O.rms_norm(0, x[:hd], w, 1, hd, 1e-6) * np.float32(40.0))


# ---- validation (no device needed: every rejection comes first) -------------------

def _msg(fn, *args):
    rc = fn(*args)
    assert rc < 0
    return si_hip.last_error()


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def test_f32_matvec_rejections():
    lib = si_hip.lib()
    x = np.zeros(4, np.float32)
    w = np.zeros(12, np.float32)
    y = np.zeros(3, np.float32)
    f = lib.si_hip_f32_matvec
    assert _msg(f, None, _fp(w), 12, 1 << 62, 1 << 62, _fp(x), 4, _fp(y)) == \
        "F32 matvec dimensions overflow"
    for rows, cols, vals, xl in [(0, 4, 0, 4), (3, 0, 0, 0), (3, 4, 11, 4), (3, 4, 12, 5)]:
        assert _msg(f, None, _fp(w), vals, rows, cols, _fp(x), xl, _fp(y)) == \
            "F32 matvec dimensions or byte length are invalid"
    assert _msg(f, None, _fp(w), 12, 3, 4, _fp(x), 4, _fp(y)) == "HIP context is null"
    fb = lib.si_hip_f32_matvec_bytes
    b = np.zeros(64, np.uint8)
    bp = b.ctypes.data_as(C.POINTER(C.c_uint8))
    assert _msg(fb, None, bp, 48, 1 << 62, 8, _fp(x), 4, _fp(y)) == \
        "F32 matvec byte length overflows"
    assert _msg(fb, None, bp, 47, 3, 4, _fp(x), 4, _fp(y)) == "F32 matvec byte length is invalid"
    odd = C.cast(C.addressof(bp.contents) + 1, C.POINTER(C.c_uint8))
    assert _msg(fb, None, odd, 48, 3, 4, _fp(x), 4, _fp(y)) == \
        "F32 matvec bytes are not 4-byte aligned"


def test_rms_norm_rejections():
    lib = si_hip.lib()
    x = np.zeros(8, np.float32)
    w = np.zeros(8, np.float32)
    y = np.zeros(8, np.float32)
    assert _msg(lib.si_hip_rms_norm, None, _fp(x), 0, _fp(w), 0, 1e-5, _fp(y)) == \
        "RMSNorm input and weight must have equal non-zero length"
    assert _msg(lib.si_hip_rms_norm, None, _fp(x), 8, _fp(w), 7, 1e-5, _fp(y)) == \
        "RMSNorm input and weight must have equal non-zero length"
    h = lib.si_hip_rms_norm_heads
    assert _msg(h, None, _fp(x), 8, _fp(w), 4, 1 << 62, 1 << 62, 1e-5, _fp(y)) == \
        "head RMSNorm dimensions overflow"
    for xl, wl, heads, hd, eps in [(8, 4, 2, 4, 0.0), (8, 4, 2, 4, -1e-6), (8, 4, 2, 4, float("nan")),
                                   (8, 4, 2, 4, float("inf")), (8, 4, 0, 4, 1e-6),
                                   (8, 4, 2, 0, 1e-6), (7, 4, 2, 4, 1e-6), (8, 3, 2, 4, 1e-6)]:
        assert _msg(h, None, _fp(x), xl, _fp(w), wl, heads, hd, eps, _fp(y)) == \
            "head RMSNorm dimensions are invalid", (xl, wl, heads, hd, eps)
    g = lib.si_hip_rms_norm_gated
    assert _msg(g, None, _fp(x), 8, _fp(x), 7, _fp(w), 4, 2, 4, 1e-6, _fp(y)) == \
        "Gated RMSNorm dimensions are invalid"
    assert _msg(g, None, _fp(x), 8, _fp(x), 8, _fp(w), 4, 1 << 62, 1 << 62, 1e-6, _fp(y)) == \
        "Gated RMSNorm dimensions overflow"
    assert _msg(g, None, _fp(x), 8, _fp(x), 8, _fp(w), 4, 2, 4, 1e-6, _fp(y)) == \
        "HIP context is null"


def _f32_store():
    rng = np.random.default_rng(21)
    a = rng.standard_normal((48, 5120)).astype(np.float32)      # [5120, 48] SSM-like matrix
    b = rng.standard_normal((6, 5120)).astype(np.float32)
    c = rng.standard_normal((5, 3)).astype(np.float32)           # 60 bytes: padded to 64
    q = bytes(2 * 144)
    tensors = [("ssm.a", [5120, 48], 0, 0, a.tobytes()),
               ("ssm.b", [5120, 6], 0, 983040, b.tobytes()),
               ("small", [3, 5], 0, 983040 + 122880, c.tobytes()),
               ("q4", [256, 2], 12, 983040 + 122880 + 64, q)]
    data, _ = write_gguf([], tensors)
    return GgufFile(data=data), a, b, c


def test_gguf_f32_rejections():
    g, a, b, c = _f32_store()
    lib = si_hip.lib()
    x = np.zeros(5120, np.float32)
    y = np.zeros(48, np.float32)
    tr = lib.si_hip_gguf_f32_matvec_tensor_rows
    assert _msg(tr, None, g.handle, g._index("q4"), 0, 1, _fp(x), 256, _fp(y)) == \
        "F32 matvec requires a rank-2 F32 tensor"
    for start, count in [(0, 0), (48, 1), (40, 9)]:
        assert _msg(tr, None, g.handle, g._index("ssm.a"), start, count, _fp(x), 5120, _fp(y)) == \
            "F32 row range is invalid"
    assert _msg(tr, None, g.handle, g._index("ssm.a"), 0, 2, _fp(x), 5119, _fp(y)) == \
        "F32 tensor columns or input length is invalid"
    assert _msg(tr, None, g.handle, g._index("ssm.a"), 0, 2, _fp(x), 5120, _fp(y)) == \
        "HIP context is null"
    many = lib.si_hip_gguf_f32_matvec_many_tensors
    outs = (C.POINTER(C.c_float) * 2)(_fp(y), _fp(y))
    idx = (C.c_uint64 * 2)(g._index("ssm.a"), g._index("small"))
    assert _msg(many, None, g.handle, idx, 0, _fp(x), 5120, outs) == \
        "GGUF F32 matvec group requires at least one tensor"
    assert _msg(many, None, g.handle, idx, 2, _fp(x), 5119, outs) == \
        "GGUF F32 matvec group input length is invalid"
    assert _msg(many, None, g.handle, idx, 2, _fp(x), 5120, outs) == \
        "GGUF F32 matvec group shapes or types differ"
    # a tensor whose range carries alignment padding is "truncated" to the reference
    idx1 = (C.c_uint64 * 1)(g._index("small"))
    assert _msg(many, None, g.handle, idx1, 1, _fp(x), 3, outs) == \
        "GGUF F32 matvec group tensor is truncated"


# ---- GPU -------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols", [(3, 4), (48, 5120), (1000, 1027), (17, 4096), (1, 1),
                                       (129, 256), (2, 17408)])
def test_f32_matvec_matches_oracle(hip_ctx, rows, cols):
    rng = np.random.default_rng(rows * 31 + cols)
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    y = hip_ctx.f32_matvec(w, rows, cols, x)
    w64, x64 = w.astype(np.float64), x.astype(np.float64)
    exact = w64 @ x64
    absdot = np.abs(w64) @ np.abs(x64)
    assert np.all(np.abs(y - exact) <= DOT_TOL * absdot + 1e-30)
    seq = O.f32_matvec(w, x, rows, cols)
    assert np.all(np.abs(y.astype(np.float64) - seq) <= 2 * DOT_TOL * absdot + 1e-30)
    yb = hip_ctx.f32_matvec_bytes(w.tobytes(), rows, cols, x)
    assert np.array_equal(y, yb)


@pytest.mark.gpu
def test_reference_f32_matvec_test(hip_ctx):
    """f32_matvec_kernel_matches_cpu_reference (src/metal.rs:7336-7361)."""
    w = np.array([1.0, 0.5, -1.0, 2.0, -2.0, 1.0, 0.25, 3.0, 0.125, -0.5, 2.0, -1.0], np.float32)
    x = np.array([2.0, -1.0, 0.5, 3.0], np.float32)
    y = hip_ctx.f32_matvec(w, 3, 4, x)
    assert np.all(np.abs(y - O.f32_matvec(w, x, 3, 4)) < 1e-5)


@pytest.mark.gpu
def test_f32_matvec_group_and_device(hip_ctx):
    rng = np.random.default_rng(5)
    cols = 3072
    mats = [rng.standard_normal((r, cols)).astype(np.float32) for r in (7, 64, 1)]
    x = rng.standard_normal(cols).astype(np.float32)
    outs = hip_ctx.f32_matvec_many(mats, [7, 64, 1], cols, x)
    for m, o in zip(mats, outs):
        assert np.array_equal(o, hip_ctx.f32_matvec(m, m.shape[0], cols, x))
    lib = si_hip.lib()
    dw = hip_ctx.device_alloc(mats[1].nbytes)
    dx = hip_ctx.device_alloc(x.nbytes)
    dy = hip_ctx.device_alloc(64 * 4)
    hip_ctx.to_device(dw, mats[1])
    hip_ctx.to_device(dx, x)
    assert lib.si_hip_f32_matvec_device(hip_ctx.handle, C.c_void_p(dw), 64, cols, C.c_void_p(dx),
                                        C.c_void_p(dy)) == 0
    hip_ctx.synchronize()
    assert np.array_equal(hip_ctx.from_device(dy, 64), outs[1])
    for p in (dw, dx, dy):
        hip_ctx.device_free(p)


@pytest.mark.gpu
def test_gguf_f32_tensor_rows_and_group(hip_ctx):
    """f32_matvec_runs_against_real_gguf_row's shape (a [5120, 48] F32 tensor,
    src/metal.rs:7704-7730) on a synthetic store: row ranges and the group."""
    g, a, b, _ = _f32_store()
    x = ((np.arange(5120) % 23).astype(np.float32) - np.float32(11.0)) / np.float32(10.0)
    for start, count in [(0, 1), (10, 20), (0, 48), (47, 1)]:
        y = g.f32_matvec_tensor_rows(hip_ctx, "ssm.a", start, count, x)
        assert np.array_equal(y, hip_ctx.f32_matvec(a[start:start + count], count, 5120, x))
    ref = O.f32_matvec(a[:1], x, 1, 5120)
    assert abs(g.f32_matvec_tensor_rows(hip_ctx, "ssm.a", 0, 1, x)[0] - ref[0]) < 1e-4
    ya, yb = g.f32_matvec_many(hip_ctx, ["ssm.a", "ssm.b"], x)
    assert np.array_equal(ya, hip_ctx.f32_matvec(a, 48, 5120, x))
    assert np.array_equal(yb, hip_ctx.f32_matvec(b, 6, 5120, x))


@pytest.mark.gpu
@pytest.mark.parametrize("mode,heads,hd", [(0, 1, 5120), (0, 1, 4), (1, 32, 128), (1, 1, 5120),
                                           (2, 48, 128), (2, 3, 7), (1, 1024, 64), (2, 1, 1)])
def test_rms_norm_matches_oracle(hip_ctx, mode, heads, hd):
    rng = np.random.default_rng(mode * 1000 + heads + hd)
    x = rng.standard_normal(heads * hd).astype(np.float32)
    w = (rng.standard_normal(hd) * 0.5).astype(np.float32)
    g = (rng.standard_normal(heads * hd) * 3).astype(np.float32)
    eps = 1e-6
    if mode == 0:
        y = hip_ctx.rms_norm(x, w, eps)
    elif mode == 1:
        y = hip_ctx.rms_norm_heads(x, w, heads, hd, eps)
    else:
        y = hip_ctx.rms_norm_gated(x, g, w, heads, hd, eps)
    ref64 = f64_rms(mode, x, w, heads, hd, eps, g)
    assert_rms_close(y, ref64, f"mode {mode}")
    oracle = O.rms_norm(mode, x, w, heads, hd, eps, gate=g if mode == 2 else None)
    assert_rms_close(oracle, ref64, "oracle")


@pytest.mark.gpu
def test_reference_rms_norm_tests(hip_ctx):
    """rms_norm / gated / head RMSNorm tests of src/metal.rs:7253-7272 and
    7412-7442, with their inputs and 1e-5 tolerance against the oracle."""
    x, w = [1.0, -2.0, 3.0, -4.0], [1.0, 0.5, 2.0, -1.0]
    assert np.all(np.abs(hip_ctx.rms_norm(x, w, 1e-5) - O.rms_norm(0, x, w, 1, 4, 1e-5)) < 1e-5)
    x, g, w = [1.0, 2.0, -1.0, 3.0], [0.0, 1.0, -1.0, 0.5], [1.0, 0.5]
    assert np.all(np.abs(hip_ctx.rms_norm_gated(x, g, w, 2, 2, 1e-6) -
                         O.rms_norm(2, x, w, 2, 2, 1e-6, gate=g)) < 1e-5)
    w = [0.25, -0.5]
    assert np.all(np.abs(hip_ctx.rms_norm_heads(x, w, 2, 2, 1e-6) -
                         O.rms_norm(1, x, w, 2, 2, 1e-6)) < 1e-5)


@pytest.mark.gpu
def test_rms_norm_device_and_extremes(hip_ctx):
    lib = si_hip.lib()
    heads, hd = 8, 96
    rng = np.random.default_rng(77)
    x = rng.standard_normal(heads * hd).astype(np.float32)
    w = rng.standard_normal(hd).astype(np.float32)
    g = np.concatenate([np.full(hd, 100.0), np.full(hd, -100.0), np.zeros(hd),
                        rng.standard_normal(5 * hd) * 20]).astype(np.float32)
    host = hip_ctx.rms_norm_gated(x, g, w, heads, hd, 1e-6)
    assert np.all(host[hd:2 * hd] == 0.0) and np.all(host[2 * hd:3 * hd] == 0.0)
    dx, dg, dw, dy = (hip_ctx.device_alloc(n * 4) for n in (heads * hd, heads * hd, hd, heads * hd))
    hip_ctx.to_device(dx, x)
    hip_ctx.to_device(dg, g)
    hip_ctx.to_device(dw, w)
    assert lib.si_hip_rms_norm_device(hip_ctx.handle, 2, C.c_void_p(dx), C.c_void_p(dg),
                                      C.c_void_p(dw), heads, hd, C.c_float(1e-6),
                                      C.c_void_p(dy)) == 0
    hip_ctx.synchronize()
    assert np.array_equal(hip_ctx.from_device(dy, heads * hd), host)
    # an infinite input: that head's mean square is infinite, its inverse 0
    xi = x.copy()
    xi[5] = np.inf
    y = hip_ctx.rms_norm_heads(xi, w, heads, hd, 1e-6)
    ref = O.rms_norm(1, xi, w, heads, hd, 1e-6)
    same = (np.isnan(y) & np.isnan(ref)) | (y == ref) | (np.abs(y - ref) <= 1e-5 * np.abs(ref))
    assert np.all(same[:hd]) and np.all(np.isfinite(y[hd:]))
    for p in (dx, dg, dw, dy):
        hip_ctx.device_free(p)
