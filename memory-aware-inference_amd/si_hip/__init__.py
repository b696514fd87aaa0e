"""Python binding of the gfx950 K-quant C ABI (include/si_hip.h).

`HipContext` mirrors the K-quant methods of super-inference's `MetalContext`
(src/metal.rs:3354-5015) with the same names and argument meaning; a
non-zero status from the C ABI raises `HipError` carrying the message the
reference would return as `Err(String)`.

The library must have been built (memory-aware-inference_amd/build.py);
there is no CPU fallback: a missing library raises at load time.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path
from typing import Iterable, Sequence

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libsi_hip.so"
INCLUDE_DIR = _HERE.parent.parent / "include"

GGML_TYPE_Q4_K = 12
GGML_TYPE_Q5_K = 13
GGML_TYPE_Q6_K = 14
BLOCK_BYTES = {GGML_TYPE_Q4_K: 144, GGML_TYPE_Q5_K: 176, GGML_TYPE_Q6_K: 210}
ARGMAX_LAST_FINITE = 0
ARGMAX_FIRST_GREATER = 1
KERNEL_AUTO = 0
KERNEL_GENERIC = 1
DEFAULT_RESIDENCY_BUDGET = 16 << 30  # SI_HIP_DEFAULT_RESIDENCY_BUDGET
MAX_BATCH = 16

STATUS = {
    0: "SI_HIP_OK", -1: "SI_HIP_ERR_NULL", -2: "SI_HIP_ERR_DIMENSIONS",
    -3: "SI_HIP_ERR_BYTE_LENGTH", -4: "SI_HIP_ERR_OVERFLOW",
    -5: "SI_HIP_ERR_UNSUPPORTED_TYPE", -6: "SI_HIP_ERR_BATCH", -7: "SI_HIP_ERR_RANGE",
    -8: "SI_HIP_ERR_NO_FINITE", -9: "SI_HIP_ERR_DEVICE", -10: "SI_HIP_ERR_OUT_OF_MEMORY",
    -11: "SI_HIP_ERR_EMPTY", -12: "SI_HIP_ERR_STATE",
}


class HipError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status
        self.message = message


class CommandStats(C.Structure):
    _fields_ = [("submitted", C.c_uint64), ("async_submitted", C.c_uint64),
                ("waited", C.c_uint64), ("wait_nanos", C.c_uint64)]


class ResidencyStats(C.Structure):
    _fields_ = [("hits", C.c_uint64), ("uploads", C.c_uint64), ("uploaded_bytes", C.c_uint64),
                ("evictions", C.c_uint64), ("resident_ranges", C.c_uint64),
                ("resident_bytes", C.c_uint64), ("budget_bytes", C.c_uint64)]


class GgufValueC(C.Structure):
    _fields_ = [("type", C.c_uint32), ("array_type", C.c_uint32), ("count", C.c_uint64),
                ("u64", C.c_uint64), ("i64", C.c_int64), ("f64", C.c_double),
                ("str", C.c_char_p), ("node", C.c_void_p)]


class GgufTensorC(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_uint32), ("ggml_type", C.c_uint32),
                ("shape", C.POINTER(C.c_uint64)), ("offset", C.c_uint64),
                ("data_start", C.c_uint64), ("data_end", C.c_uint64)]


_P = C.c_void_p
_SZ = C.c_size_t
_U32 = C.c_uint32
_U64 = C.c_uint64
_I = C.c_int
_FP = C.POINTER(C.c_float)
_BP = C.POINTER(C.c_uint8)
_U32P = C.POINTER(C.c_uint32)

# name -> (restype, argtypes)
_SIGS = {
    "si_hip_last_error": (C.c_char_p, []),
    "si_hip_status_name": (C.c_char_p, [_I]),
    "si_hip_abi_version": (_U32, []),
    "si_hip_context_new": (_I, [_I, C.POINTER(_P)]),
    "si_hip_context_free": (None, [_P]),
    "si_hip_upload_quant_weight_private": (_I, [_P, _BP, _SZ, _U32, C.POINTER(_P)]),
    "si_hip_bind_quant_weight_mapped": (_I, [_P, _BP, _SZ, _U32, C.POINTER(_P)]),
    "si_hip_quant_weight_view": (_I, [_P, _U64, _U64, _U32, C.POINTER(_P)]),
    "si_hip_quant_weight_free": (None, [_P]),
    "si_hip_quant_weight_byte_len": (_U64, [_P]),
    "si_hip_quant_weight_ggml_type": (_U32, [_P]),
    "si_hip_quant_weight_is_mapped": (_I, [_P]),
    "si_hip_quant_weight_device_ptr": (_P, [_P]),
    "si_hip_q4_k_matvec": (_I, [_P, _BP, _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_q5_k_matvec": (_I, [_P, _BP, _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_q6_k_matvec": (_I, [_P, _BP, _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_gguf_quant_matvec_bytes": (_I, [_P, _U32, _BP, _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_gguf_quant_matvec_weight": (_I, [_P, _P, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_gguf_quant_matvec_tensor_rows": (_I, [_P, _P, _SZ, _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_gguf_quant_matvec_many_weights": (
        _I, [_P, C.POINTER(_P), C.POINTER(_SZ), _SZ, _SZ, _FP, _SZ, C.POINTER(_FP)]),
    "si_hip_q4_k_fused_gate_up": (_I, [_P, _BP, _SZ, _BP, _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_q4_k_fused_gate_up_weights": (_I, [_P, _P, _P, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_gguf_quant_fused_mlp_weights": (_I, [_P, _P, _P, _P, _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_q4_k_embedding_row": (_I, [_P, _BP, _SZ, _SZ, _FP]),
    "si_hip_q4_k_embedding_view": (_I, [_P, _U32, C.POINTER(_U64), _U32, _BP, _SZ, _SZ, _FP]),
    "si_hip_gguf_quant_matvec_view_rows": (_I, [_P, C.c_char_p, _U32, C.POINTER(_U64), _U32, _BP,
                                                _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_q4_k_embedding_tensor": (_I, [_P, _P, _SZ, _SZ, _SZ, _FP]),
    "si_hip_q4_k_embedding_tokens": (_I, [_P, _P, _SZ, _SZ, _U32P, _SZ, _FP]),
    "si_hip_gguf_quant_matmul_many_bytes": (_I, [_P, _U32, _BP, _SZ, _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_gguf_quant_matmul_many_weight": (_I, [_P, _P, _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_gguf_quant_matvec_argmax_weight": (_I, [_P, _P, _SZ, _SZ, _FP, _SZ, _U32, _U32P, _FP]),
    "si_hip_dequantize": (_I, [_P, _U32, _BP, _SZ, _SZ, _FP]),
    "si_hip_device_alloc": (_I, [_P, _SZ, C.POINTER(_P)]),
    "si_hip_device_free": (_I, [_P, _P]),
    "si_hip_copy_to_device": (_I, [_P, _P, _P, _SZ]),
    "si_hip_copy_from_device": (_I, [_P, _P, _P, _SZ]),
    "si_hip_copy_device": (_I, [_P, _P, _P, _SZ]),
    "si_hip_synchronize": (_I, [_P]),
    "si_hip_quant_matvec_device": (_I, [_P, _P, _SZ, _SZ, _P, _P]),
    "si_hip_quant_matvec_many_device": (_I, [_P, C.POINTER(_P), C.POINTER(_SZ), _SZ, _SZ, _P,
                                             _P]),
    "si_hip_q4_k_fused_gate_up_device": (_I, [_P, _P, _P, _SZ, _SZ, _P, _P]),
    "si_hip_fused_mlp_device": (_I, [_P, _P, _P, _P, _SZ, _SZ, _SZ, _P, _P, _P]),
    "si_hip_matmul_many_device": (_I, [_P, _P, _SZ, _SZ, _SZ, _P, _P]),
    "si_hip_matvec_argmax_device": (_I, [_P, _P, _SZ, _SZ, _P, _U32, _P, _P]),
    "si_hip_argmax_result_index": (_U32, [_U64, _U32]),
    "si_hip_embedding_device": (_I, [_P, _P, _SZ, _SZ, _P, _SZ, _P]),
    "si_hip_event_record": (_I, [_P, _U32]),
    "si_hip_event_elapsed_ms": (_I, [_P, _U32, _U32, C.POINTER(C.c_float)]),
    "si_hip_quant_matvec_device_repeat": (_I, [_P, C.POINTER(_P), _SZ, _SZ, _SZ, _P, _P, _SZ]),
    "si_hip_stream_probe": (_I, [_P, C.POINTER(_P), _SZ, _SZ, _SZ, _U32, _SZ]),
    "si_hip_capture_begin": (_I, [_P]),
    "si_hip_capture_end": (_I, [_P, C.POINTER(_P)]),
    "si_hip_graph_launch": (_I, [_P, _P]),
    "si_hip_graph_calls": (_U64, [_P]),
    "si_hip_graph_free": (None, [_P]),
    "si_hip_set_kernel_policy": (_I, [_P, _U32]),
    "si_hip_debug_set_wait_give_up": (_I, [_P, _U32]),
    "si_hip_current_allocated_bytes": (_U64, [_P]),
    "si_hip_peak_allocated_bytes": (_U64, [_P]),
    "si_hip_peak_active_weight_bytes": (_U64, [_P]),
    "si_hip_reset_peaks": (None, [_P]),
    "si_hip_sample_allocated": (None, [_P]),
    "si_hip_get_command_stats": (_I, [_P, C.POINTER(CommandStats)]),
    "si_hip_set_residency_budget": (_I, [_P, _U64]),
    "si_hip_residency_evict": (_I, [_P, _P, _SZ]),
    "si_hip_get_residency_stats": (_I, [_P, C.POINTER(ResidencyStats)]),
    # si_hip_f32.h
    "si_hip_f32_matvec": (_I, [_P, _FP, _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_f32_matvec_bytes": (_I, [_P, _BP, _SZ, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_f32_matvec_many": (_I, [_P, C.POINTER(_FP), C.POINTER(_SZ), _SZ, _SZ, _FP, _SZ,
                                    C.POINTER(_FP)]),
    "si_hip_f32_matvec_device": (_I, [_P, _P, _SZ, _SZ, _P, _P]),
    "si_hip_rms_norm": (_I, [_P, _FP, _SZ, _FP, _SZ, C.c_float, _FP]),
    "si_hip_rms_norm_heads": (_I, [_P, _FP, _SZ, _FP, _SZ, _SZ, _SZ, C.c_float, _FP]),
    "si_hip_rms_norm_gated": (_I, [_P, _FP, _SZ, _FP, _SZ, _FP, _SZ, _SZ, _SZ, C.c_float, _FP]),
    "si_hip_rms_norm_device": (_I, [_P, _U32, _P, _P, _P, _SZ, _SZ, C.c_float, _P]),
    "si_hip_gguf_f32_matvec_tensor_rows": (_I, [_P, _P, _U64, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_gguf_f32_matvec_many_tensors": (_I, [_P, _P, C.POINTER(_U64), _SZ, _FP, _SZ,
                                                 C.POINTER(_FP)]),
    "si_hip_gguf_matvec_tensor_rows": (_I, [_P, _P, _U64, _SZ, _SZ, _FP, _SZ, _FP]),
    "si_hip_gguf_quant_matvec_many_tensors": (_I, [_P, _P, C.POINTER(_U64), _SZ, _FP, _SZ,
                                                   C.POINTER(_FP)]),
    "si_hip_gguf_quant_matvec_many_bytes": (
        _I, [_P, C.POINTER(C.c_uint32), C.POINTER(_BP), C.POINTER(_SZ), C.POINTER(_SZ),
             C.POINTER(_SZ), _SZ, _FP, _SZ, C.POINTER(_FP)]),
    # si_hip_gguf.h
    "si_hip_gguf_open": (_I, [C.c_char_p, C.POINTER(_P)]),
    "si_hip_gguf_parse": (_I, [_BP, _SZ, C.POINTER(_P)]),
    "si_hip_gguf_close": (None, [_P]),
    "si_hip_gguf_version": (_U32, [_P]),
    "si_hip_gguf_alignment": (_U64, [_P]),
    "si_hip_gguf_data_base": (_U64, [_P]),
    "si_hip_gguf_file_bytes": (_U64, [_P]),
    "si_hip_gguf_tensor_count": (_U64, [_P]),
    "si_hip_gguf_tensor_info": (_I, [_P, _U64, C.POINTER(GgufTensorC)]),
    "si_hip_gguf_find_tensor": (_I, [_P, C.c_char_p, C.POINTER(_U64)]),
    "si_hip_gguf_tensor_data": (_I, [_P, _U64, C.POINTER(_BP), C.POINTER(_U64)]),
    "si_hip_gguf_tensor_elements": (_I, [_P, _U64, C.POINTER(_U64)]),
    "si_hip_gguf_expected_payload_bytes": (_I, [_P, _U64, C.POINTER(_U64), C.POINTER(_I)]),
    "si_hip_gguf_metadata_count": (_U64, [_P]),
    "si_hip_gguf_metadata_key": (_I, [_P, _U64, C.POINTER(C.c_char_p)]),
    "si_hip_gguf_metadata_get": (_I, [_P, C.c_char_p, C.POINTER(GgufValueC)]),
    "si_hip_gguf_value_item": (_I, [C.POINTER(GgufValueC), _U64, C.POINTER(GgufValueC)]),
    "si_hip_gguf_upload_tensor": (_I, [_P, _P, _U64, C.POINTER(_P)]),
    "si_hip_gguf_bind_tensor_mapped": (_I, [_P, _P, _U64, C.POINTER(_P)]),
    # si_hip_synth.h
    "si_hip_synth_blocks": (_I, [_U32, _U64, _U64, _SZ, _BP, _SZ, _I]),
    "si_hip_synth_normal_f32": (_I, [_U64, _U64, _SZ, C.c_float, _FP]),
    "si_hip_synth_token_ids": (_I, [_U64, _SZ, _U32, _U32P]),
    "si_hip_quant_matvec_noalloc": (_I, [_U32, C.c_void_p, _SZ, _SZ, _SZ, C.c_void_p,
                                         C.c_void_p, C.c_void_p]),
    "si_hip_noalloc_check": (_I, [C.c_void_p]),
    "si_hip_noalloc_debug_set_wait_give_up": (_I, [_U32, C.c_void_p]),
    "si_hip_synth_f32_to_f16": (C.c_uint16, [C.c_float]),
}

_lib = None


def lib() -> C.CDLL:
    """Load libsi_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with "
                "`python memory-aware-inference_amd/build.py` (no CPU fallback exists)")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def header_symbols() -> list[str]:
    """Every function the public headers declare."""
    names = []
    for h in sorted(INCLUDE_DIR.glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"\b(si_hip_\w+)\s*\(", text)
    return sorted(set(names))


def last_error() -> str:
    return lib().si_hip_last_error().decode()


def _check(status: int) -> None:
    if status != 0:
        raise HipError(status, last_error())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_FP)


def _u8(b) -> np.ndarray:
    if isinstance(b, (bytes, bytearray, memoryview)):
        return np.frombuffer(b, dtype=np.uint8)
    return np.ascontiguousarray(b, dtype=np.uint8)


def _bp(a: np.ndarray):
    return a.ctypes.data_as(_BP)


# ---------------------------------------------------------------------------
# synthetic data (host only, no GPU needed)

def synth_blocks(ggml_type: int, seed: int, n_blocks: int, first_block: int = 0,
                 threads: int = 1) -> np.ndarray:
    out = np.empty(n_blocks * BLOCK_BYTES[ggml_type], dtype=np.uint8)
    _check(lib().si_hip_synth_blocks(ggml_type, seed, first_block, n_blocks, _bp(out), out.size,
                                     threads))
    return out


def synth_matrix(ggml_type: int, seed: int, rows: int, cols: int, threads: int = 1) -> np.ndarray:
    return synth_blocks(ggml_type, seed, rows * (cols // 256), threads=threads)


def synth_normal(seed: int, n: int, scale: float = 1.0, first_index: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _check(lib().si_hip_synth_normal_f32(seed, first_index, n, scale, _fp(out)))
    return out


def synth_token_ids(seed: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    _check(lib().si_hip_synth_token_ids(seed, n, vocab, out.ctypes.data_as(_U32P)))
    return out


def f32_to_f16_bits(v: float) -> int:
    return int(lib().si_hip_synth_f32_to_f16(v))


# ---------------------------------------------------------------------------

class QuantWeight:
    """Owning handle of HBM-resident packed blocks (QuantWeight, metal.rs:1840)."""

    def __init__(self, ctx: "HipContext", handle: int, parent: "QuantWeight | None" = None):
        self._ctx = ctx
        self._h = C.c_void_p(handle)
        self._parent = parent

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def byte_len(self) -> int:
        return int(lib().si_hip_quant_weight_byte_len(self._h))

    def ggml_type(self) -> int:
        return int(lib().si_hip_quant_weight_ggml_type(self._h))

    def is_mapped(self) -> bool:
        return bool(lib().si_hip_quant_weight_is_mapped(self._h))

    def device_ptr(self) -> int:
        return int(lib().si_hip_quant_weight_device_ptr(self._h) or 0)

    def view(self, offset: int, nbytes: int, ggml_type: int) -> "QuantWeight":
        out = C.c_void_p()
        _check(lib().si_hip_quant_weight_view(self._h, offset, nbytes, ggml_type, C.byref(out)))
        return QuantWeight(self._ctx, out.value, parent=self)

    def free(self) -> None:
        if self._h:
            lib().si_hip_quant_weight_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HipGraph:
    """Device calls recorded by HipContext.capture_begin/capture_end."""

    def __init__(self, ctx: "HipContext", handle: C.c_void_p):
        self._ctx = ctx
        self.handle = handle

    @property
    def calls(self) -> int:
        return int(lib().si_hip_graph_calls(self.handle))

    def launch(self) -> None:
        _check(lib().si_hip_graph_launch(self._ctx._h, self.handle))

    def free(self) -> None:
        if self.handle:
            lib().si_hip_graph_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HipContext:
    """K-quant surface of MetalContext on one MI355X GPU."""

    def __init__(self, device: int = 0):
        out = C.c_void_p()
        _check(lib().si_hip_context_new(device, C.byref(out)))
        self._h = out

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def close(self) -> None:
        if self._h:
            lib().si_hip_context_free(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def set_kernel_policy(self, policy: int) -> None:
        _check(lib().si_hip_set_kernel_policy(self._h, policy))

    def debug_set_wait_give_up(self, polls: int) -> None:
        """Test hook: the kernels' bounded waits give up after `polls` polls
        (0 restores normal waits)."""
        _check(lib().si_hip_debug_set_wait_give_up(self._h, polls))

    # ---- weights
    def upload_quant_weight_private(self, weight_bytes, ggml_type: int) -> QuantWeight:
        b = _u8(weight_bytes)
        out = C.c_void_p()
        _check(lib().si_hip_upload_quant_weight_private(self._h, _bp(b), b.size, ggml_type,
                                                        C.byref(out)))
        return QuantWeight(self, out.value)

    def bind_quant_weight_mapped(self, weight_bytes, ggml_type: int) -> QuantWeight:
        b = _u8(weight_bytes)
        out = C.c_void_p()
        _check(lib().si_hip_bind_quant_weight_mapped(self._h, _bp(b), b.size, ggml_type,
                                                     C.byref(out)))
        return QuantWeight(self, out.value)

    # ---- matvec
    def _typed(self, fn, weight_bytes, rows, columns, input) -> np.ndarray:
        b, x = _u8(weight_bytes), _f32(input)
        y = np.empty(rows, dtype=np.float32)
        _check(fn(self._h, _bp(b), b.size, rows, columns, _fp(x), x.size, _fp(y)))
        return y

    def q4_k_matvec(self, weight_bytes, rows: int, columns: int, input) -> np.ndarray:
        return self._typed(lib().si_hip_q4_k_matvec, weight_bytes, rows, columns, input)

    def q5_k_matvec(self, weight_bytes, rows: int, columns: int, input) -> np.ndarray:
        return self._typed(lib().si_hip_q5_k_matvec, weight_bytes, rows, columns, input)

    def q6_k_matvec(self, weight_bytes, rows: int, columns: int, input) -> np.ndarray:
        return self._typed(lib().si_hip_q6_k_matvec, weight_bytes, rows, columns, input)

    def gguf_quant_matvec_bytes(self, ggml_type: int, weight_bytes, rows: int, columns: int,
                                input) -> np.ndarray:
        b, x = _u8(weight_bytes), _f32(input)
        y = np.empty(rows, dtype=np.float32)
        _check(lib().si_hip_gguf_quant_matvec_bytes(self._h, ggml_type, _bp(b), b.size, rows,
                                                    columns, _fp(x), x.size, _fp(y)))
        return y

    def gguf_quant_matvec_weight(self, weight: QuantWeight, rows: int, columns: int,
                                 input) -> np.ndarray:
        x = _f32(input)
        y = np.empty(rows, dtype=np.float32)
        _check(lib().si_hip_gguf_quant_matvec_weight(self._h, weight.handle, rows, columns,
                                                     _fp(x), x.size, _fp(y)))
        return y

    def gguf_quant_matvec_tensor_rows(self, tensor: QuantWeight, shape: Sequence[int],
                                      row_start: int, row_count: int, input) -> np.ndarray:
        x = _f32(input)
        y = np.empty(max(row_count, 1), dtype=np.float32)
        _check(lib().si_hip_gguf_quant_matvec_tensor_rows(
            self._h, tensor.handle, shape[0], shape[1], row_start, row_count, _fp(x), x.size,
            _fp(y)))
        return y[:row_count]

    def gguf_quant_matvec_many_weights(self, weights: Sequence[QuantWeight],
                                       rows: Sequence[int], columns: int, input) -> list:
        x = _f32(input)
        n = len(weights)
        outs = [np.empty(r, dtype=np.float32) for r in rows]
        harr = (C.c_void_p * n)(*[w.handle.value for w in weights])
        rarr = (C.c_size_t * n)(*rows)
        oarr = (_FP * n)(*[_fp(o) for o in outs])
        _check(lib().si_hip_gguf_quant_matvec_many_weights(self._h, harr, rarr, n, columns,
                                                           _fp(x), x.size, oarr))
        return outs

    def gguf_quant_matvec_many_bytes(self, tensors: Sequence, input) -> list:
        """gguf_quant_matvec_many_bytes (src/metal.rs:4878-5001): tensors are
        (ggml_type, bytes, rows, columns); one result per tensor."""
        x = _f32(input)
        n = len(tensors)
        arrs = [_u8(b) for (_, b, _, _) in tensors]
        outs = [np.empty(max(int(r), 1), dtype=np.float32) for (_, _, r, _) in tensors]
        types = (C.c_uint32 * n)(*[int(t) for (t, _, _, _) in tensors])
        bp = (_BP * n)(*[_bp(a) for a in arrs])
        lens = (C.c_size_t * n)(*[a.size for a in arrs])
        rows = (C.c_size_t * n)(*[int(r) for (_, _, r, _) in tensors])
        cols = (C.c_size_t * n)(*[int(c) for (_, _, _, c) in tensors])
        oarr = (_FP * n)(*[_fp(o) for o in outs])
        _check(lib().si_hip_gguf_quant_matvec_many_bytes(self._h, types, bp, lens, rows, cols, n,
                                                         _fp(x), x.size, oarr))
        return outs

    def quant_matvec_many_device(self, weights: Sequence[QuantWeight], rows: Sequence[int],
                                 columns: int, d_input: int, d_output: int) -> None:
        """Device-resident grouped matvec: weight i's rows land in d_output
        after those of the weights before it (enqueued; synchronize() waits)."""
        n = len(weights)
        harr = (C.c_void_p * n)(*[w.handle.value for w in weights])
        rarr = (C.c_size_t * n)(*rows)
        _check(lib().si_hip_quant_matvec_many_device(self._h, harr, rarr, n, columns,
                                                     C.c_void_p(d_input), C.c_void_p(d_output)))

    # ---- fused SwiGLU
    def q4_k_fused_gate_up(self, gate_bytes, up_bytes, rows: int, columns: int,
                           input) -> np.ndarray:
        g, u, x = _u8(gate_bytes), _u8(up_bytes), _f32(input)
        y = np.empty(rows, dtype=np.float32)
        _check(lib().si_hip_q4_k_fused_gate_up(self._h, _bp(g), g.size, _bp(u), u.size, rows,
                                               columns, _fp(x), x.size, _fp(y)))
        return y

    def q4_k_fused_gate_up_weights(self, gate: QuantWeight, up: QuantWeight, rows: int,
                                   columns: int, input) -> np.ndarray:
        x = _f32(input)
        y = np.empty(rows, dtype=np.float32)
        _check(lib().si_hip_q4_k_fused_gate_up_weights(self._h, gate.handle, up.handle, rows,
                                                       columns, _fp(x), x.size, _fp(y)))
        return y

    def gguf_quant_fused_mlp_weights(self, gate: QuantWeight, up: QuantWeight,
                                     down: QuantWeight, gate_rows: int, columns: int,
                                     down_rows: int, input) -> np.ndarray:
        x = _f32(input)
        y = np.empty(down_rows, dtype=np.float32)
        _check(lib().si_hip_gguf_quant_fused_mlp_weights(
            self._h, gate.handle, up.handle, down.handle, gate_rows, columns, down_rows, _fp(x),
            x.size, _fp(y)))
        return y

    # ---- embedding
    def q4_k_embedding_row(self, row_bytes, columns: int) -> np.ndarray:
        b = _u8(row_bytes)
        y = np.empty(max(columns, 1), dtype=np.float32)
        _check(lib().si_hip_q4_k_embedding_row(self._h, _bp(b), b.size, columns, _fp(y)))
        return y[:columns]

    def q4_k_embedding_view(self, ggml_type: int, shape: Sequence[int], payload,
                            token_id: int) -> np.ndarray:
        """q4_k_embedding_tensor over a GgufTensorView (type, shape, borrowed
        payload bytes)."""
        b = _u8(payload)
        sh = (_U64 * len(shape))(*shape)
        y = np.empty(max(int(shape[0]) if shape else 1, 1), dtype=np.float32)
        _check(lib().si_hip_q4_k_embedding_view(self._h, ggml_type, sh, len(shape), _bp(b), b.size,
                                                token_id, _fp(y)))
        return y[:int(shape[0])]

    def gguf_quant_matvec_view_rows(self, name: str, ggml_type: int, shape: Sequence[int],
                                    payload, row_start: int, row_count: int, input) -> np.ndarray:
        """gguf_quant_matvec_tensor_rows over a GgufTensorView."""
        b, x = _u8(payload), _f32(input)
        sh = (_U64 * len(shape))(*shape)
        y = np.empty(max(row_count, 1), dtype=np.float32)
        _check(lib().si_hip_gguf_quant_matvec_view_rows(self._h, name.encode(), ggml_type, sh,
                                                        len(shape), _bp(b), b.size, row_start,
                                                        row_count, _fp(x), x.size, _fp(y)))
        return y[:row_count]

    def q4_k_embedding_tensor(self, table: QuantWeight, shape: Sequence[int],
                              token_id: int) -> np.ndarray:
        y = np.empty(max(shape[0], 1), dtype=np.float32)
        _check(lib().si_hip_q4_k_embedding_tensor(self._h, table.handle, shape[0], shape[1],
                                                  token_id, _fp(y)))
        return y[:shape[0]]

    def q4_k_embedding_tokens(self, table: QuantWeight, shape: Sequence[int],
                              token_ids) -> np.ndarray:
        ids = np.ascontiguousarray(token_ids, dtype=np.uint32)
        y = np.empty((max(ids.size, 1), shape[0]), dtype=np.float32)
        _check(lib().si_hip_q4_k_embedding_tokens(self._h, table.handle, shape[0], shape[1],
                                                  ids.ctypes.data_as(_U32P), ids.size, _fp(y)))
        return y[:ids.size]

    # ---- multi-token verify (the reference's Vec<Vec<f32>>, batch-major)
    def gguf_quant_matmul_many_bytes(self, ggml_type: int, weight_bytes, rows: int, columns: int,
                                     batch: int, inputs) -> list:
        b, x = _u8(weight_bytes), _f32(inputs).reshape(-1)
        y = np.empty(max(batch, 1) * rows, dtype=np.float32)
        _check(lib().si_hip_gguf_quant_matmul_many_bytes(self._h, ggml_type, _bp(b), b.size, rows,
                                                         columns, batch, _fp(x), x.size, _fp(y)))
        return [y[i * rows:(i + 1) * rows] for i in range(batch)]

    def gguf_quant_matmul_many_weight(self, weight: QuantWeight, rows: int, columns: int,
                                      batch: int, inputs) -> list:
        x = _f32(inputs).reshape(-1)
        y = np.empty(max(batch, 1) * rows, dtype=np.float32)
        _check(lib().si_hip_gguf_quant_matmul_many_weight(self._h, weight.handle, rows, columns,
                                                          batch, _fp(x), x.size, _fp(y)))
        return [y[i * rows:(i + 1) * rows] for i in range(batch)]

    # ---- head + argmax
    def gguf_quant_matvec_argmax_weight(self, head: QuantWeight, rows: int, columns: int, input,
                                        rule: int = ARGMAX_LAST_FINITE,
                                        want_logits: bool = True):
        x = _f32(input)
        tok = C.c_uint32()
        logits = np.empty(rows, dtype=np.float32) if want_logits else None
        _check(lib().si_hip_gguf_quant_matvec_argmax_weight(
            self._h, head.handle, rows, columns, _fp(x), x.size, rule, C.byref(tok),
            _fp(logits) if logits is not None else None))
        return int(tok.value), logits

    # ---- F32 matvec and RMSNorm (include/si_hip_f32.h) ----
    def f32_matvec(self, weight_values, rows: int, columns: int, input) -> np.ndarray:
        w = _f32(weight_values).reshape(-1)
        x = _f32(input)
        y = np.empty(max(rows, 1), dtype=np.float32)
        _check(lib().si_hip_f32_matvec(self._h, _fp(w), w.size, rows, columns, _fp(x), x.size,
                                       _fp(y)))
        return y[:rows]

    def f32_matvec_bytes(self, weight_bytes, rows: int, columns: int, input) -> np.ndarray:
        b = _u8(weight_bytes)
        x = _f32(input)
        y = np.empty(max(rows, 1), dtype=np.float32)
        _check(lib().si_hip_f32_matvec_bytes(self._h, _bp(b), b.size, rows, columns, _fp(x),
                                             x.size, _fp(y)))
        return y[:rows]

    def f32_matvec_many(self, weights: Sequence, rows: Sequence[int], columns: int,
                        input) -> list:
        ws = [_f32(w).reshape(-1) for w in weights]
        x = _f32(input)
        ys = [np.empty(max(r, 1), dtype=np.float32) for r in rows]
        wp = (_FP * len(ws))(*[_fp(w) for w in ws])
        yp = (_FP * len(ys))(*[_fp(y) for y in ys])
        rp = (C.c_size_t * len(rows))(*rows)
        _check(lib().si_hip_f32_matvec_many(self._h, wp, rp, len(ws), columns, _fp(x), x.size,
                                            yp))
        return [y[:r] for y, r in zip(ys, rows)]

    def rms_norm(self, input, weight, epsilon: float) -> np.ndarray:
        x, w = _f32(input), _f32(weight)
        y = np.empty(max(x.size, 1), dtype=np.float32)
        _check(lib().si_hip_rms_norm(self._h, _fp(x), x.size, _fp(w), w.size, epsilon, _fp(y)))
        return y[:x.size]

    def rms_norm_heads(self, input, weight, heads: int, head_dim: int,
                       epsilon: float) -> np.ndarray:
        x, w = _f32(input), _f32(weight)
        y = np.empty(max(x.size, 1), dtype=np.float32)
        _check(lib().si_hip_rms_norm_heads(self._h, _fp(x), x.size, _fp(w), w.size, heads,
                                           head_dim, epsilon, _fp(y)))
        return y[:x.size]

    def rms_norm_gated(self, input, gate, weight, heads: int, head_dim: int,
                       epsilon: float) -> np.ndarray:
        x, g, w = _f32(input), _f32(gate), _f32(weight)
        y = np.empty(max(x.size, 1), dtype=np.float32)
        _check(lib().si_hip_rms_norm_gated(self._h, _fp(x), x.size, _fp(g), g.size, _fp(w),
                                           w.size, heads, head_dim, epsilon, _fp(y)))
        return y[:x.size]

    def dequantize(self, ggml_type: int, data, elements: int) -> np.ndarray:
        b = _u8(data)
        y = np.empty(max(elements, 1), dtype=np.float32)
        _check(lib().si_hip_dequantize(self._h, ggml_type, _bp(b), b.size, elements, _fp(y)))
        return y[:elements]

    # ---- device-resident plumbing
    def device_alloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        _check(lib().si_hip_device_alloc(self._h, nbytes, C.byref(p)))
        return p.value

    def device_copy(self, dst: int, src: int, nbytes: int) -> None:
        _check(lib().si_hip_copy_device(self._h, C.c_void_p(dst), C.c_void_p(src), nbytes))

    def device_free(self, ptr: int) -> None:
        _check(lib().si_hip_device_free(self._h, C.c_void_p(ptr)))

    def to_device(self, ptr: int, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        _check(lib().si_hip_copy_to_device(self._h, C.c_void_p(ptr), a.ctypes.data_as(_P),
                                           a.nbytes))

    def from_device(self, ptr: int, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        _check(lib().si_hip_copy_from_device(self._h, out.ctypes.data_as(_P), C.c_void_p(ptr),
                                             out.nbytes))
        return out

    def synchronize(self) -> None:
        _check(lib().si_hip_synchronize(self._h))

    def event_record(self, slot: int) -> None:
        _check(lib().si_hip_event_record(self._h, slot))

    def event_elapsed_ms(self, a: int, b: int) -> float:
        ms = C.c_float()
        _check(lib().si_hip_event_elapsed_ms(self._h, a, b, C.byref(ms)))
        return float(ms.value)

    # ---- captured submission
    def capture_begin(self) -> None:
        """Record the following *_device calls into a graph instead of running them."""
        _check(lib().si_hip_capture_begin(self._h))

    def capture_end(self) -> "HipGraph":
        g = C.c_void_p()
        _check(lib().si_hip_capture_end(self._h, C.byref(g)))
        return HipGraph(self, g)

    # ---- telemetry
    def current_allocated_bytes(self) -> int:
        return int(lib().si_hip_current_allocated_bytes(self._h))

    def peak_allocated_bytes(self) -> int:
        return int(lib().si_hip_peak_allocated_bytes(self._h))

    def peak_active_weight_bytes(self) -> int:
        return int(lib().si_hip_peak_active_weight_bytes(self._h))

    def reset_peaks(self) -> None:
        lib().si_hip_reset_peaks(self._h)

    def sample_allocated(self) -> None:
        """sample_allocated (src/metal.rs:2374-2378): peak = max(peak, current)."""
        lib().si_hip_sample_allocated(self._h)

    def command_stats(self) -> dict:
        s = CommandStats()
        _check(lib().si_hip_get_command_stats(self._h, C.byref(s)))
        return {k: int(getattr(s, k)) for k, _ in CommandStats._fields_}

    # ---- residency of borrowed weight bytes
    def set_residency_budget(self, nbytes: int) -> None:
        _check(lib().si_hip_set_residency_budget(self._h, nbytes))

    def residency_evict(self, host_bytes=None, nbytes: int = 0) -> None:
        """Drops resident ranges overlapping the buffer (None: every range)."""
        if host_bytes is None:
            _check(lib().si_hip_residency_evict(self._h, None, 0))
            return
        b = _u8(host_bytes)
        _check(lib().si_hip_residency_evict(self._h, b.ctypes.data_as(_P), nbytes or b.size))

    def residency_stats(self) -> dict:
        s = ResidencyStats()
        _check(lib().si_hip_get_residency_stats(self._h, C.byref(s)))
        return {k: int(getattr(s, k)) for k, _ in ResidencyStats._fields_}

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- GGUF model store (include/si_hip_gguf.h) ---------------------------------
GGUF_TYPE_NAMES = ("U8", "I8", "U16", "I16", "U32", "I32", "F32", "Bool", "String", "Array",
                   "U64", "I64", "F64")


class GgufValue:
    """A metadata value with its GGUF type (GgufValue, src/model.rs:304-318)."""

    __slots__ = ("type", "value")

    def __init__(self, type_: int, value):
        self.type = type_
        self.value = value

    def __eq__(self, other):
        if not isinstance(other, GgufValue):
            return NotImplemented
        return self.type == other.type and self.value == other.value

    def __repr__(self):
        """Rust's derived Debug form: U32(32), F32(1e-6), String("qwen35")."""
        if self.type in (6, 12):
            body = _debug_float(self.value, self.type == 6)
        elif self.type == 7:
            body = "true" if self.value else "false"
        elif self.type == 8:
            body = _debug_str(self.value)
        elif self.type == 9:
            body = "[" + ", ".join(repr(v) for v in self.value) + "]"
        else:
            body = str(self.value)
        return f"{GGUF_TYPE_NAMES[self.type]}({body})"


def _debug_float(v: float, single: bool) -> str:
    """Debug formatting of an f32/f64: shortest round-trip digits, positional
    with at least one fractional digit for 1e-4 <= |v| < 1e16 (and zero),
    scientific ("1e-6", "1.5e16") otherwise."""
    if v != v:
        return "NaN"
    if v in (float("inf"), float("-inf")):
        return "inf" if v > 0 else "-inf"
    x = np.float32(v) if single else np.float64(v)
    a = abs(float(v))
    if a == 0.0 or 1e-4 <= a < 1e16:
        return np.format_float_positional(x, unique=True, trim="0")
    mant, exp = np.format_float_scientific(x, unique=True, trim="-").split("e")
    return f"{mant}e{int(exp)}"


def _debug_str(v: str) -> str:
    """A string in Rust's Debug form: double quotes, backslash escapes for
    quote, backslash, tab, CR, LF and NUL, \\u{..} for other unprintables."""
    out = ['"']
    for ch in v:
        if ch in '"\\':
            out.append("\\" + ch)
        elif ch == "\n":
            out.append("\\n")
        elif ch == "\r":
            out.append("\\r")
        elif ch == "\t":
            out.append("\\t")
        elif ch == "\0":
            out.append("\\0")
        elif not ch.isprintable():
            out.append("\\u{%x}" % ord(ch))
        else:
            out.append(ch)
    out.append('"')
    return "".join(out)


def _gguf_value(v: GgufValueC) -> GgufValue:
    t = v.type
    if t in (0, 2, 4, 10):
        return GgufValue(t, int(v.u64))
    if t in (1, 3, 5, 11):
        return GgufValue(t, int(v.i64))
    if t in (6, 12):
        return GgufValue(t, float(v.f64))
    if t == 7:
        return GgufValue(t, bool(v.u64))
    if t == 8:
        return GgufValue(t, C.string_at(v.str, v.count).decode("utf-8"))
    items = []
    for i in range(v.count):
        it = GgufValueC()
        _check(lib().si_hip_gguf_value_item(C.byref(v), i, C.byref(it)))
        items.append(_gguf_value(it))
    return GgufValue(t, items)


class GgufTensorInfo:
    """One tensor of a GGUF index (GgufTensorInfo, src/model.rs:498-505)."""

    __slots__ = ("index", "name", "shape", "ggml_type", "offset", "data_start", "data_end")

    def __init__(self, index, name, shape, ggml_type, offset, data_start, data_end):
        self.index, self.name, self.shape, self.ggml_type = index, name, shape, ggml_type
        self.offset, self.data_start, self.data_end = offset, data_start, data_end

    def byte_len(self) -> int:
        return self.data_end - self.data_start

    def element_count(self) -> int | None:
        """The product of the dimensions, None when it overflows 64 bits
        (the reference's "element count overflows" error)."""
        n = 1
        for d in self.shape:
            n *= d
            if n >= 1 << 64:
                return None
        return n

    def is_q4_k(self) -> bool:
        return self.ggml_type == GGML_TYPE_Q4_K


class GgufFile:
    """GgufModelStore (src/model.rs:583-681) over the C store: a read-only
    mapping of the file (or a copy of given bytes), its metadata and tensor
    index, tensor byte views and uploads of K-quant tensors to HBM."""

    def __init__(self, path: str | os.PathLike | None = None, data: bytes | None = None):
        h = C.c_void_p()
        if (path is None) == (data is None):
            raise ValueError("give exactly one of path and data")
        if path is not None:
            _check(lib().si_hip_gguf_open(os.fsencode(path), C.byref(h)))
        else:
            b = _u8(data)
            _check(lib().si_hip_gguf_parse(_bp(b), b.size, C.byref(h)))
        self._h = h
        self.path = None if path is None else str(path)
        n = int(lib().si_hip_gguf_tensor_count(h))
        self.tensor_list = []
        for i in range(n):
            t = GgufTensorC()
            _check(lib().si_hip_gguf_tensor_info(h, i, C.byref(t)))
            self.tensor_list.append(GgufTensorInfo(
                i, t.name.decode("utf-8"), tuple(t.shape[k] for k in range(t.n_dims)),
                t.ggml_type, t.offset, t.data_start, t.data_end))
        # name -> info; a repeated name keeps its last tensor, like the reference's map
        self.tensors = {t.name: t for t in self.tensor_list}
        self.metadata = {}
        for i in range(int(lib().si_hip_gguf_metadata_count(h))):
            key = C.c_char_p()
            _check(lib().si_hip_gguf_metadata_key(h, i, C.byref(key)))
            v = GgufValueC()
            _check(lib().si_hip_gguf_metadata_get(h, key.value, C.byref(v)))
            self.metadata[key.value.decode("utf-8")] = _gguf_value(v)

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    @property
    def version(self) -> int:
        return int(lib().si_hip_gguf_version(self._h))

    @property
    def alignment(self) -> int:
        return int(lib().si_hip_gguf_alignment(self._h))

    @property
    def data_base(self) -> int:
        return int(lib().si_hip_gguf_data_base(self._h))

    def _index(self, name: str) -> int:
        i = C.c_uint64()
        _check(lib().si_hip_gguf_find_tensor(self._h, name.encode("utf-8"), C.byref(i)))
        return int(i.value)

    def tensor(self, name: str) -> tuple[GgufTensorInfo, np.ndarray]:
        """GgufModelStore::tensor: the info and a copy of the tensor's bytes."""
        i = self._index(name)
        p = C.POINTER(C.c_uint8)()
        n = C.c_uint64()
        _check(lib().si_hip_gguf_tensor_data(self._h, i, C.byref(p), C.byref(n)))
        data = np.ctypeslib.as_array(p, shape=(int(n.value),)).copy() if n.value else \
            np.empty(0, np.uint8)
        return self.tensor_list[i], data

    def element_count(self, name: str) -> int:
        out = C.c_uint64()
        _check(lib().si_hip_gguf_tensor_elements(self._h, self._index(name), C.byref(out)))
        return int(out.value)

    def expected_payload_bytes(self, name: str) -> int | None:
        out, known = C.c_uint64(), C.c_int()
        _check(lib().si_hip_gguf_expected_payload_bytes(self._h, self._index(name), C.byref(out),
                                                        C.byref(known)))
        return int(out.value) if known.value else None

    def upload(self, ctx: "HipContext", name: str, mapped: bool = False) -> "QuantWeight":
        """The K-quant tensor's payload as a QuantWeight in HBM."""
        w = C.c_void_p()
        fn = lib().si_hip_gguf_bind_tensor_mapped if mapped else lib().si_hip_gguf_upload_tensor
        _check(fn(ctx.handle, self._h, self._index(name), C.byref(w)))
        return QuantWeight(ctx, w.value)

    def f32_matvec_tensor_rows(self, ctx: "HipContext", name: str, row_start: int,
                               row_count: int, input) -> np.ndarray:
        """f32_matvec_tensor_rows (src/metal.rs:3074-3110) on this store's tensor."""
        x = _f32(input)
        y = np.empty(max(row_count, 1), dtype=np.float32)
        _check(lib().si_hip_gguf_f32_matvec_tensor_rows(ctx.handle, self._h, self._index(name),
                                                        row_start, row_count, _fp(x), x.size,
                                                        _fp(y)))
        return y[:row_count]

    def f32_matvec_many(self, ctx: "HipContext", names: Sequence[str], input) -> list:
        """f32_matvec_many_gguf_tensors (src/metal.rs:4780-4870): one result per tensor."""
        x = _f32(input)
        idx = [self._index(n) for n in names]
        ys = [np.empty(max(int(self.tensor_list[i].shape[1]), 1) if len(self.tensor_list[i].shape) == 2
                       else 1, dtype=np.float32) for i in idx]
        yp = (_FP * len(ys))(*[_fp(y) for y in ys])
        ip = (C.c_uint64 * len(idx))(*idx)
        _check(lib().si_hip_gguf_f32_matvec_many_tensors(ctx.handle, self._h, ip, len(idx), _fp(x),
                                                         x.size, yp))
        return ys

    def matvec_tensor_rows(self, ctx: "HipContext", name: str, row_start: int, row_count: int,
                           input) -> np.ndarray:
        """gguf_matvec_tensor_rows (src/metal.rs:5003-5015): F32 or K-quant rows."""
        x = _f32(input)
        y = np.empty(max(row_count, 1), dtype=np.float32)
        _check(lib().si_hip_gguf_matvec_tensor_rows(ctx.handle, self._h, self._index(name),
                                                    row_start, row_count, _fp(x), x.size,
                                                    _fp(y)))
        return y[:row_count]

    def quant_matvec_many(self, ctx: "HipContext", names: Sequence[str], input) -> list:
        """gguf_quant_matvec_many_tensors (src/metal.rs:4532-4646): one result per tensor."""
        x = _f32(input)
        idx = [self._index(n) for n in names]
        ys = [np.empty(max(int(self.tensor_list[i].shape[1]), 1) if len(self.tensor_list[i].shape) == 2
                       else 1, dtype=np.float32) for i in idx]
        yp = (_FP * len(ys))(*[_fp(y) for y in ys])
        ip = (C.c_uint64 * len(idx))(*idx)
        _check(lib().si_hip_gguf_quant_matvec_many_tensors(ctx.handle, self._h, ip, len(idx),
                                                           _fp(x), x.size, yp))
        return ys

    def inspect(self, model: str | None = None) -> str:
        """The dump si-gguf-inspect prints (src/bin/si-gguf-inspect.rs:11-60)."""
        lines = [f"model={model or self.path}", f"tensors={len(self.tensors)}"]
        by_name = sorted(self.tensors.values(), key=lambda t: t.name.encode("utf-8"))
        for t in [t for t in by_name if t.is_q4_k()][:12]:
            lines.append(f"q4_k_tensor={t.name} shape={list(t.shape)} bytes={t.byte_len()} "
                         f"elements={t.element_count() or 0}")
        counts = {}
        for t in by_name:
            counts[t.ggml_type] = counts.get(t.ggml_type, 0) + 1
        lines.append("tensor_type_counts={" + ", ".join(
            f"{k}: {v}" for k, v in sorted(counts.items())) + "}")
        for name in ("token_embd.weight", "output.weight", "output_norm.weight"):
            t = self.tensors.get(name)
            if t is not None:
                lines.append(f"special_tensor={name} type={t.ggml_type} shape={list(t.shape)} "
                             f"bytes={t.byte_len()}")
        for t in [t for t in by_name if not t.is_q4_k()][:24]:
            lines.append(f"non_q4_tensor={t.name} type={t.ggml_type} shape={list(t.shape)} "
                         f"bytes={t.byte_len()}")
        for key in sorted(self.metadata, key=lambda k: k.encode("utf-8")):
            lines.append(f"metadata.{key}={_summarize(self.metadata[key])}")
        return "\n".join(lines)

    def close(self) -> None:
        if self._h:
            lib().si_hip_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _summarize(v: GgufValue) -> str:
    """summarize() of si-gguf-inspect (src/bin/si-gguf-inspect.rs:86-101)."""
    if v.type == 9:
        preview = ", ".join(_summarize(x) for x in v.value[:3])
        return f"array(len={len(v.value)}, first=[{preview}])"
    if v.type == 8:
        if len(v.value.encode("utf-8")) > 160:
            return f"string(len={len(v.value.encode('utf-8'))}, prefix={_debug_str(v.value[:160])})"
        return f"string({_debug_str(v.value)})"
    return repr(v)
