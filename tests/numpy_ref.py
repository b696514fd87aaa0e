"""Second, independent restatement of src/quant.rs in vectorised numpy.

Test infrastructure only.  Structured differently from oracle/kquant_ref.c
(whole arrays of blocks at once instead of per-element loops) so that an
indexing or ordering slip in either one shows up as a bit mismatch.  numpy
float32 arithmetic rounds every operation and never contracts, matching the
separately rounded f32 steps of quant.rs.
"""
from __future__ import annotations

import numpy as np

BLOCK = {12: 144, 13: 176, 14: 210}


def _blocks(data, block_bytes: int) -> np.ndarray:
    a = np.frombuffer(bytes(data), dtype=np.uint8) if not isinstance(data, np.ndarray) else data
    return a.reshape(-1, block_bytes)


def _half(raw2: np.ndarray) -> np.ndarray:
    """Two little-endian bytes per row -> float32 via numpy's float16."""
    return np.ascontiguousarray(raw2).view("<f2").astype(np.float32).reshape(-1)


def _k4_scales(s: np.ndarray):
    """quant.rs:176-185 over a (n, 12) array -> (n, 8) scales and mins."""
    s = s.astype(np.uint32)
    sc = np.empty((s.shape[0], 8), dtype=np.uint32)
    mn = np.empty_like(sc)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc.astype(np.float32), mn.astype(np.float32)


def dequant_q4_k(data) -> np.ndarray:
    b = _blocks(data, 144)
    n = b.shape[0]
    d, dmin = _half(b[:, 0:2]), _half(b[:, 2:4])
    sc, mn = _k4_scales(b[:, 4:16])
    d1 = d[:, None] * sc        # (n, 8)
    m1 = dmin[:, None] * mn
    q = b[:, 16:144].reshape(n, 4, 32)
    out = np.empty((n, 4, 2, 32), dtype=np.float32)
    out[:, :, 0, :] = d1[:, 0::2, None] * (q & 15).astype(np.float32) - m1[:, 0::2, None]
    out[:, :, 1, :] = d1[:, 1::2, None] * (q >> 4).astype(np.float32) - m1[:, 1::2, None]
    return out.reshape(-1)


def dequant_q5_k(data) -> np.ndarray:
    b = _blocks(data, 176)
    n = b.shape[0]
    d, dmin = _half(b[:, 0:2]), _half(b[:, 2:4])
    sc, mn = _k4_scales(b[:, 4:16])
    d1 = d[:, None] * sc
    m1 = dmin[:, None] * mn
    qh = b[:, 16:48].astype(np.uint32)                       # (n, 32)
    q = b[:, 48:176].reshape(n, 4, 32).astype(np.uint32)
    g = np.arange(4, dtype=np.uint32)[None, :, None]
    lo = (q & 15) + 16 * ((qh[:, None, :] >> (2 * g)) & 1)
    hi = (q >> 4) + 16 * ((qh[:, None, :] >> (2 * g + 1)) & 1)
    out = np.empty((n, 4, 2, 32), dtype=np.float32)
    out[:, :, 0, :] = d1[:, 0::2, None] * lo.astype(np.float32) - m1[:, 0::2, None]
    out[:, :, 1, :] = d1[:, 1::2, None] * hi.astype(np.float32) - m1[:, 1::2, None]
    return out.reshape(-1)


def dequant_q6_k(data) -> np.ndarray:
    b = _blocks(data, 210)
    n = b.shape[0]
    d = _half(b[:, 208:210])
    sc = b[:, 192:208].view(np.int8).astype(np.float32)        # (n, 16)
    out = np.empty((n, 2, 4, 32), dtype=np.float32)
    i = np.arange(32)
    for h in range(2):
        ql = b[:, 64 * h:64 * h + 64].astype(np.int32)
        qh = b[:, 128 + 32 * h:160 + 32 * h].astype(np.int32)
        quads = [
            (ql[:, :32] & 15) | ((qh & 3) << 4),
            (ql[:, 32:] & 15) | (((qh >> 2) & 3) << 4),
            (ql[:, :32] >> 4) | (((qh >> 4) & 3) << 4),
            (ql[:, 32:] >> 4) | ((qh >> 6) << 4),
        ]
        for k, qv in enumerate(quads):
            s = sc[:, 8 * h + (i // 16) + 2 * k]               # (n, 32)
            out[:, h, k, :] = (d[:, None] * s) * (qv - 32).astype(np.float32)
    return out.reshape(-1)


def dequant(ggml_type: int, data) -> np.ndarray:
    with np.errstate(invalid="ignore", over="ignore"):
        return {12: dequant_q4_k, 13: dequant_q5_k, 14: dequant_q6_k}[ggml_type](data)


def encode_k4_scales(sc, mn) -> bytes:
    """Pack eight 6-bit scales and eight 6-bit mins into GGML's 12 bytes.

    Written from the format description (bytes 0-3: scales 0-3 in bits 0-5,
    bits 6-7 carry bits 4-5 of scales 4-7; bytes 4-7: the same for mins;
    bytes 8-11: low nibble = bits 0-3 of scale j+4, high nibble = bits 0-3 of
    min j+4), so a round trip through the decoder checks get_scale_min.
    """
    out = bytearray(12)
    for j in range(4):
        out[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return bytes(out)
