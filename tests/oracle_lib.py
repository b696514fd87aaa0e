"""ctypes access to the CPU oracle (oracle/kquant_ref.c): the checker only."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent.parent
ORACLE_SO = REPO / "oracle" / "_build" / "libkquant_ref.so"

KQ_OK = 0
KQ_ERR_ELEMENTS = -1
KQ_ERR_BYTES = -2
KQ_ERR_OVERFLOW = -3
KQ_ERR_TYPE = -4
KQ_ERR_NO_FINITE = -5

_FP = C.POINTER(C.c_float)
_DP = C.POINTER(C.c_double)
_BP = C.POINTER(C.c_uint8)
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(REPO / "oracle")], check=True)
    return ORACLE_SO


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            build()
        h = C.CDLL(str(ORACLE_SO))
        h.kq_f16_to_f32.restype = C.c_float
        h.kq_f16_to_f32.argtypes = [C.c_uint16]
        h.kq_f16_to_f32_bits.restype = C.c_uint32
        h.kq_f16_to_f32_bits.argtypes = [C.c_uint16]
        h.kq_get_scale_min.restype = None
        h.kq_get_scale_min.argtypes = [C.c_uint, _BP, _BP, _BP]
        for name in ("kq_dequantize_q4_k", "kq_dequantize_q5_k", "kq_dequantize_q6_k"):
            fn = getattr(h, name)
            fn.restype = C.c_int
            fn.argtypes = [_BP, C.c_size_t, C.c_size_t, _FP]
        h.kq_dequantize.restype = C.c_int
        h.kq_dequantize.argtypes = [C.c_uint32, _BP, C.c_size_t, C.c_size_t, _FP]
        h.kq_dot_f32_sequential.restype = C.c_float
        h.kq_dot_f32_sequential.argtypes = [_FP, _FP, C.c_size_t]
        h.kq_dot_f64.restype = C.c_double
        h.kq_dot_f64.argtypes = [_FP, _FP, C.c_size_t]
        h.kq_abs_dot_f64.restype = C.c_double
        h.kq_abs_dot_f64.argtypes = [_FP, _FP, C.c_size_t]
        h.kq_matvec_ref.restype = C.c_int
        h.kq_matvec_ref.argtypes = [C.c_uint32, _BP, C.c_size_t, C.c_size_t, C.c_size_t, _FP,
                                    _FP, _DP, _DP, C.c_int]
        h.kq_silu.restype = C.c_float
        h.kq_silu.argtypes = [C.c_float]
        h.kq_argmax_last_finite.restype = C.c_int
        h.kq_argmax_last_finite.argtypes = [_FP, C.c_size_t, C.POINTER(C.c_uint32)]
        h.kq_argmax_first_greater.restype = C.c_uint32
        h.kq_argmax_first_greater.argtypes = [_FP, C.c_size_t]
        h.kq_f32_matvec_ref.restype = C.c_int
        h.kq_f32_matvec_ref.argtypes = [_FP, _FP, C.c_size_t, C.c_size_t, _FP]
        h.kq_rms_norm_ref.restype = C.c_int
        h.kq_rms_norm_ref.argtypes = [C.c_uint32, _FP, _FP, _FP, C.c_size_t, C.c_size_t,
                                      C.c_float, _FP]
        _lib = h
    return _lib


def _u8(b):
    a = np.ascontiguousarray(np.frombuffer(b, dtype=np.uint8) if isinstance(b, (bytes, bytearray))
                             else b, dtype=np.uint8)
    return a


def dequantize(ggml_type: int, data, elements: int) -> np.ndarray:
    a = _u8(data)
    out = np.empty(max(elements, 1), dtype=np.float32)
    rc = lib().kq_dequantize(ggml_type, a.ctypes.data_as(_BP), a.size, elements,
                             out.ctypes.data_as(_FP))
    if rc != KQ_OK:
        raise ValueError(f"oracle dequantize rejected input (code {rc})")
    return out[:elements]


def dequantize_rc(ggml_type: int, data, elements: int) -> int:
    a = _u8(data)
    out = np.empty(max(elements, 256), dtype=np.float32)
    return lib().kq_dequantize(ggml_type, a.ctypes.data_as(_BP), a.size, elements,
                               out.ctypes.data_as(_FP))


def matvec(ggml_type: int, data, rows: int, cols: int, x, threads: int = 1):
    """(y_f32 sequential, y_f64, sum|w*x| f64) per row."""
    a = _u8(data)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y32 = np.empty(rows, dtype=np.float32)
    y64 = np.empty(rows, dtype=np.float64)
    ab = np.empty(rows, dtype=np.float64)
    rc = lib().kq_matvec_ref(ggml_type, a.ctypes.data_as(_BP), a.size, rows, cols,
                             x.ctypes.data_as(_FP), y32.ctypes.data_as(_FP),
                             y64.ctypes.data_as(_DP), ab.ctypes.data_as(_DP), threads)
    if rc != KQ_OK:
        raise ValueError(f"oracle matvec rejected input (code {rc})")
    return y32, y64, ab


def f16_to_f32(bits: int) -> float:
    return lib().kq_f16_to_f32(bits)


def f16_to_f32_bits(bits: int) -> int:
    return int(lib().kq_f16_to_f32_bits(bits))


def get_scale_min(index: int, scales: bytes) -> tuple[int, int]:
    s = (C.c_uint8 * 12)(*scales)
    sc, mn = C.c_uint8(), C.c_uint8()
    lib().kq_get_scale_min(index, s, C.byref(sc), C.byref(mn))
    return sc.value, mn.value


def silu(v: float) -> float:
    return lib().kq_silu(v)


def argmax_last_finite(v) -> int | None:
    a = np.ascontiguousarray(v, dtype=np.float32)
    idx = C.c_uint32()
    rc = lib().kq_argmax_last_finite(a.ctypes.data_as(_FP), a.size, C.byref(idx))
    return None if rc == KQ_ERR_NO_FINITE else int(idx.value)


def argmax_first_greater(v) -> int:
    a = np.ascontiguousarray(v, dtype=np.float32)
    return int(lib().kq_argmax_first_greater(a.ctypes.data_as(_FP), a.size))


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_FP)


def f32_matvec(w, x, rows: int, cols: int) -> np.ndarray:
    """Sequential-f32 F32 matvec of the reference's test (oracle/f32_ref.c)."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(rows, dtype=np.float32)
    assert lib().kq_f32_matvec_ref(_fp(w), _fp(x), rows, cols, _fp(out)) == 0
    return out


def rms_norm(mode: int, x, w, heads: int, head_dim: int, eps: float, gate=None) -> np.ndarray:
    """RMSNorm of oracle/f32_ref.c: mode 0 (x*inv*w), 1 (x*inv*(1+w)), 2 (gated)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    g = np.ascontiguousarray(gate if gate is not None else np.zeros(1), dtype=np.float32)
    out = np.empty(heads * head_dim, dtype=np.float32)
    assert lib().kq_rms_norm_ref(mode, _fp(x), _fp(g) if gate is not None else None, _fp(w),
                                 heads, head_dim, eps, _fp(out)) == 0
    return out
