"""C-ABI library checks that need no GPU: symbols, host-side validation
(every rejection fires before the context is touched, as in the reference,
so ctx = NULL is enough), and the synthetic-data generator."""
import ctypes as C

import numpy as np
import pytest

import si_hip
from si_hip import lib

NULL = None


def status_of(fn, *args):
    return fn(*args)


def test_library_exports_every_header_symbol():
    names = si_hip.header_symbols()
    assert len(names) > 50
    handle = lib()
    missing = [n for n in names if not hasattr(handle, n)]
    assert missing == []
    # and the Python binding declares a signature for each of them
    assert sorted(set(names) - set(si_hip._SIGS)) == []
    assert lib().si_hip_abi_version() == 1


def _x(n):
    return np.zeros(n, dtype=np.float32)


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _bp(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint8))


def matvec_status(fn, wlen, rows, cols, xlen):
    w = np.zeros(max(wlen, 1), dtype=np.uint8)
    x = _x(max(xlen, 1))
    y = _x(max(rows, 1))
    return fn(NULL, _bp(w), wlen, rows, cols, _fp(x), xlen, _fp(y))


@pytest.mark.parametrize("name,bb", [("si_hip_q4_k_matvec", 144), ("si_hip_q5_k_matvec", 176),
                                     ("si_hip_q6_k_matvec", 210)])
def test_matvec_rejections_match_reference_order(name, bb):
    fn = getattr(lib(), name)
    label = {144: "Q4_K", 176: "Q5_K", 210: "Q6_K"}[bb]
    # metal.rs:3847-3849: rows/cols zero, cols % 256, input length
    for rows, cols, xlen in [(0, 256, 256), (1, 0, 0), (1, 255, 255), (1, 512, 256)]:
        assert matvec_status(fn, bb, rows, cols, xlen) == -2
        assert si_hip.last_error() == f"{label} matvec dimensions are invalid"
    # metal.rs:3856-3858: byte length
    assert matvec_status(fn, 2 * bb - 1, 2, 256, 256) == -3
    assert si_hip.last_error() == f"{label} matvec byte length is invalid"
    assert matvec_status(fn, 2 * bb + 1, 2, 256, 256) == -3
    # valid shape but no context
    assert matvec_status(fn, 2 * bb, 2, 256, 256) == -1


def test_matvec_bytes_unsupported_type_and_overflow():
    L = lib()
    w, x, y = np.zeros(16, np.uint8), _x(256), _x(1)
    assert L.si_hip_gguf_quant_matvec_bytes(NULL, 2, _bp(w), 16, 1, 256, _fp(x), 256, _fp(y)) == -5
    assert si_hip.last_error() == "unsupported staged quantized weight type"
    # rows * (cols/256) * 144 overflows size_t
    huge = (1 << 63)
    assert L.si_hip_q4_k_matvec(NULL, _bp(w), 16, huge, 512, _fp(x), 512, _fp(y)) == -4


def test_rows_beyond_u32_rejected():
    L = lib()
    rows = (1 << 32) + 1
    w, x, y = np.zeros(1, np.uint8), _x(256), _x(1)
    assert L.si_hip_q4_k_matvec(NULL, _bp(w), rows * 144, rows, 256, _fp(x), 256, _fp(y)) == -4
    assert "rows exceed HIP limits" in si_hip.last_error()


def test_fused_gate_up_rejections():
    L = lib()
    g = np.zeros(288, np.uint8)
    x, y = _x(256), _x(2)
    f = L.si_hip_q4_k_fused_gate_up
    assert f(NULL, _bp(g), 288, _bp(g), 288, 0, 256, _fp(x), 256, _fp(y)) == -2
    assert si_hip.last_error() == "Q4_K fused gate/up dimensions are invalid"
    assert f(NULL, _bp(g), 288, _bp(g), 287, 2, 256, _fp(x), 256, _fp(y)) == -3
    assert si_hip.last_error() == "Q4_K fused gate/up byte length is invalid"
    assert f(NULL, _bp(g), 288, _bp(g), 288, 2, 256, _fp(x), 256, _fp(y)) == -1


def test_matmul_many_batch_bounds():
    L = lib()
    w = np.zeros(144, np.uint8)
    x = _x(17 * 256)
    y = _x(17)
    f = L.si_hip_gguf_quant_matmul_many_bytes
    for batch in (0, 17):
        assert f(NULL, 12, _bp(w), 144, 1, 256, batch, _fp(x), batch * 256, _fp(y)) == -6
        assert si_hip.last_error() == "batched quantized matvec dimensions are invalid"
    assert f(NULL, 12, _bp(w), 144, 1, 256, 2, _fp(x), 3 * 256, _fp(y)) == -2
    assert si_hip.last_error() == "batched quantized input length is invalid"
    assert f(NULL, 9, _bp(w), 144, 1, 256, 2, _fp(x), 512, _fp(y)) == -5
    assert f(NULL, 12, _bp(w), 143, 1, 256, 2, _fp(x), 512, _fp(y)) == -3
    assert f(NULL, 12, _bp(w), 144, 1, 256, 16, _fp(x), 16 * 256, _fp(y)) == -1


_BP = C.POINTER(C.c_uint8)
_FP = C.POINTER(C.c_float)


def test_grouped_bytes_rejections():
    """gguf_quant_matvec_many_bytes's checks, in its order (metal.rs:4878-4935)."""
    L = lib()
    w = np.zeros(2 * 144, np.uint8)
    x, y = _x(256), _x(4)
    f = L.si_hip_gguf_quant_matvec_many_bytes

    def call(types, lens, rows, cols, n=None, xl=256):
        n = len(types) if n is None else n
        return f(NULL, (C.c_uint32 * max(n, 1))(*types), (_BP * max(n, 1))(*[_bp(w)] * max(n, 1)),
                 (C.c_size_t * max(n, 1))(*lens), (C.c_size_t * max(n, 1))(*rows),
                 (C.c_size_t * max(n, 1))(*cols), n, _fp(x), xl,
                 (_FP * max(n, 1))(*[_fp(y)] * max(n, 1)))

    assert call([12], [144], [1], [256], n=0) == -11
    assert si_hip.last_error() == "staged quantized matvec group requires at least one tensor"
    assert call([12], [144], [1], [256], xl=255) == -2
    assert si_hip.last_error() == "staged quantized matvec group input length is invalid"
    assert call([12, 12], [144, 144], [1, 1], [256, 512]) == -2
    assert si_hip.last_error() == "staged quantized matvec group shapes differ"
    assert call([12, 12], [144, 144], [1, 0], [256, 256]) == -2
    assert call([12, 9], [144, 144], [1, 1], [256, 256]) == -5
    assert si_hip.last_error() == "unsupported staged quantized tensor type"
    assert call([12, 13], [144, 144], [1, 1], [256, 256]) == -3
    assert si_hip.last_error() == "staged quantized matvec tensor byte length is invalid"
    assert call([12, 12], [144, 288], [1, 2], [256, 256]) == -1  # valid: the context is null


def test_embedding_row_and_dequantize_rejections():
    L = lib()
    w = np.zeros(288, np.uint8)
    y = _x(512)
    assert L.si_hip_q4_k_embedding_row(NULL, _bp(w), 144, 0, _fp(y)) == -2
    assert si_hip.last_error() == "Q4_K embedding dimension is invalid"
    assert L.si_hip_q4_k_embedding_row(NULL, _bp(w), 143, 256, _fp(y)) == -3
    assert si_hip.last_error() == "Q4_K embedding row byte length is invalid"
    # quant.rs:233-238 restated for the GPU dequantiser
    assert L.si_hip_dequantize(NULL, 12, _bp(w), 144, 255, _fp(y)) == -2
    assert L.si_hip_dequantize(NULL, 12, _bp(w), 143, 256, _fp(y)) == -3
    assert L.si_hip_dequantize(NULL, 12, _bp(w), 145, 256, _fp(y)) == -3
    assert si_hip.last_error() == "Q4_K data has 145 bytes; expected 144"
    assert L.si_hip_dequantize(NULL, 7, _bp(w), 144, 256, _fp(y)) == -5


def _shape(*dims):
    return (C.c_uint64 * len(dims))(*dims), len(dims)


def test_view_rows_rejections_match_reference_order():
    """gguf_quant_matvec_tensor_rows then quant_k_matvec_tensor_rows
    (src/metal.rs:4346-4527): each check, in the reference's order, on a
    GgufTensorView given as (name, type, shape, payload)."""
    L = lib()
    w = np.zeros(10 * 144 * 4, np.uint8)
    x = _x(1024)
    y = _x(16)

    def call(t, shape, payload_len, start, count, xl=1024, name=b"blk.0.ffn_up.weight"):
        sh, n = shape
        rc = L.si_hip_gguf_quant_matvec_view_rows(NULL, name, t, sh, n, _bp(w), payload_len, start,
                                                  count, _fp(x), xl, _fp(y))
        return rc, si_hip.last_error()

    assert call(2, _shape(1024, 10), w.size, 0, 1) == (
        -5, "GGUF tensor blk.0.ffn_up.weight has unsupported quantized type 2")
    assert call(12, _shape(1024, 10, 1), w.size, 0, 1) == (
        -5, "Q4_K matvec requires a rank-2 Q4_K tensor")
    assert call(14, _shape(1024, 10), w.size, 10, 1) == (-7, "Q6_K row range is invalid")
    assert call(13, _shape(1024, 10), w.size, 3, 8) == (-7, "Q5_K row range is invalid")
    assert call(12, _shape(1024, 10), w.size, 0, 0) == (-7, "Q4_K row range is invalid")
    assert call(12, _shape(1000, 10), w.size, 0, 1) == (
        -2, "Q4_K tensor columns or input length is invalid")
    assert call(12, _shape(1024, 10), w.size, 0, 1, xl=1023) == (
        -2, "Q4_K tensor columns or input length is invalid")
    # a payload that holds rows 0..8 of 10: row 9 is past it, rows 0..8 pass the
    # checks (and then need a context)
    assert call(12, _shape(1024, 10), 9 * 576, 9, 1) == (
        -3, "Q4_K tensor payload is shorter than its shape")
    assert call(12, _shape(1024, 10), 9 * 576, 0, 9)[0] == -1
    big = (1 << 64) // 576 + 1
    assert call(12, _shape(1024, big + 5), w.size, big, 1) == (
        -4, "Q4_K row byte range overflows")


def test_embedding_view_rejections_match_reference_order():
    """q4_k_embedding_tensor (src/metal.rs:3785-3810), then
    q4_k_embedding_row's dimension check: a table shorter than its shape
    still serves the rows it holds."""
    L = lib()
    t = np.zeros(16 * 144, np.uint8)
    y = _x(256)

    def call(ty, shape, payload_len, token):
        sh, n = shape
        rc = L.si_hip_q4_k_embedding_view(NULL, ty, sh, n, _bp(t), payload_len, token, _fp(y))
        return rc, si_hip.last_error()

    assert call(14, _shape(256, 16), t.size, 0) == (-5, "Q4_K embedding requires a rank-2 Q4_K tensor")
    assert call(12, _shape(256, 16, 1), t.size, 0) == (
        -5, "Q4_K embedding requires a rank-2 Q4_K tensor")
    assert call(12, _shape(256, 16), t.size, 16) == (-7, "Q4_K embedding token id or dimension is invalid")
    assert call(12, _shape(257, 16), t.size, 0) == (-7, "Q4_K embedding token id or dimension is invalid")
    assert call(12, _shape(256, 16), 10 * 144, 12) == (
        -3, "Q4_K embedding tensor payload is shorter than its shape")
    assert call(12, _shape(256, 16), 10 * 144, 9)[0] == -1  # held: reaches the context check
    assert call(12, _shape(0, 16), t.size, 0) == (-2, "Q4_K embedding dimension is invalid")
    big = (1 << 64) // 576  # 1024 columns: 576-byte rows
    assert call(12, _shape(1024, big * 2), t.size, big + 1) == (
        -4, "Q4_K embedding row offset overflows")
    assert call(12, _shape(1024, big * 2), t.size, big) == (-4, "Q4_K embedding row end overflows")


def test_weight_upload_rejections_without_gpu():
    L = lib()
    out = C.c_void_p()
    w = np.zeros(144, np.uint8)
    assert L.si_hip_upload_quant_weight_private(NULL, _bp(w), 0, 12, C.byref(out)) == -11
    assert si_hip.last_error() == "unsupported or empty quantized weight"
    assert L.si_hip_upload_quant_weight_private(NULL, _bp(w), 144, 1, C.byref(out)) == -5
    assert L.si_hip_bind_quant_weight_mapped(NULL, _bp(w), 144, 15, C.byref(out)) == -5
    assert si_hip.last_error() == "unsupported or empty mapped quantized weight"
    assert L.si_hip_upload_quant_weight_private(NULL, _bp(w), 144, 12, C.byref(out)) == -1


def test_status_names():
    assert lib().si_hip_status_name(-3) == b"SI_HIP_ERR_BYTE_LENGTH"
    assert lib().si_hip_status_name(0) == b"SI_HIP_OK"


# ---- synthetic data ------------------------------------------------------------
def test_synth_is_counter_based_and_thread_invariant():
    a = si_hip.synth_blocks(12, seed=5, n_blocks=5000, threads=1)
    b = si_hip.synth_blocks(12, seed=5, n_blocks=5000, threads=8)
    assert np.array_equal(a, b)
    c = si_hip.synth_blocks(12, seed=5, n_blocks=10, first_block=1234)
    assert np.array_equal(c, a[1234 * 144:1244 * 144])
    assert not np.array_equal(si_hip.synth_blocks(12, seed=6, n_blocks=10), a[:1440])


def test_synth_f16_converter_matches_numpy():
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
                           np.array([0.0, -0.0, 65504.0, 65520.0, 65519.0, 2 ** -24, 2 ** -25, 2 ** -26,
                                     3 * 2 ** -26, 1e-8, np.inf, -np.inf], np.float32)]).astype(np.float32)
    ours = np.array([si_hip.f32_to_f16_bits(float(v)) for v in vals], dtype=np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_synth_block_statistics():
    n = 50000
    q4 = si_hip.synth_blocks(12, seed=77, n_blocks=n).reshape(n, 144)
    d = q4[:, 0:2].copy().view("<f2").astype(np.float64).ravel()
    dmin = q4[:, 2:4].copy().view("<f2").astype(np.float64).ravel()
    for v in (d, dmin):
        assert np.all(v >= 0)
        assert abs(v.mean() - 0.02 * np.sqrt(2 / np.pi)) < 5e-4      # E|N(0, s)| = s*sqrt(2/pi)
        sub = np.mean(v < 2.0 ** -14)                                   # f16 subnormal share
        assert 0.0010 < sub < 0.0040
    assert abs(q4[:, 16:].mean() - 127.5) < 0.5
    q6 = si_hip.synth_blocks(14, seed=78, n_blocks=n).reshape(n, 210)
    sc = q6[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31
    d6 = q6[:, 208:210].copy().view("<f2").astype(np.float64).ravel()
    assert abs(d6.mean() - 0.01 * np.sqrt(2 / np.pi)) < 3e-4


def test_synth_normal_and_token_ids():
    x = si_hip.synth_normal(1, 200000)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert np.array_equal(si_hip.synth_normal(1, 10, first_index=7), x[7:17])
    ids = si_hip.synth_token_ids(3, 10000, 151936)
    assert ids.max() < 151936 and len(np.unique(ids)) > 9000
