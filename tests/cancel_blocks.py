"""Q4_K / Q5_K matrices whose weights cancel inside their own decode.

quant.rs decodes a Q4_K weight as d * sc * q - dmin * m (quant.rs:45-59) and a
Q5_K one the same way with 5-bit q (quant.rs:107-121).  With dmin == d and
m == sc * q* for each unit, every quant equal to q* decodes to exactly 0: the
two products are exact in f32 (an f16 times a 6-bit integer times at most 5
more bits) and equal, so their difference is 0.  Row kinds, by row index mod 4:

  0  every weight of the row cancels (the reference's dot is exactly 0)
  1  about 1 % of the quants differ from q* (99 % of the weights cancel)
  2  about 10 % differ
  3  an ordinary row of the seeded generator (si_hip.synth_matrix)

d (== dmin) is |N(0, 0.02)| rounded to f16, q* uniform in 1..QMAX and sc
uniform in 1..63 // q*, per block and unit.
"""
from __future__ import annotations

import numpy as np

import si_hip

Q4, Q5 = 12, 13
ROW_KINDS = 4
FLIP = {0: 0.0, 1: 0.005, 2: 0.05}  # fraction of quant bytes replaced by random ones


def _scale_bytes(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """GGML's 12 scale bytes of eight 6-bit scales and mins, per block
    (the packing numpy_ref.encode_k4_scales writes, vectorised)."""
    out = np.empty(sc.shape[:-1] + (12,), np.uint8)
    for j in range(4):
        out[..., j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        out[..., j + 4] = (mn[..., j] & 63) | ((mn[..., j + 4] >> 4) << 6)
        out[..., j + 8] = (sc[..., j + 4] & 15) | ((mn[..., j + 4] & 15) << 4)
    return out


def matrix(ggml_type: int, rows: int, cols: int, seed: int) -> bytes:
    """rows x cols packed Q4_K (12) or Q5_K (13) bytes with the row kinds above."""
    assert ggml_type in (Q4, Q5) and cols % 256 == 0
    nb = cols // 256
    rng = np.random.default_rng(seed)
    qmax = 15 if ggml_type == Q4 else 31
    bb = 144 if ggml_type == Q4 else 176
    nblk = rows * nb
    d = np.abs(rng.normal(0.0, 0.02, nblk)).astype(np.float16)
    d[d == 0] = np.float16(0.01)
    qstar = rng.integers(1, qmax + 1, (nblk, 8)).astype(np.int64)
    sc = rng.integers(1, 63 // qstar + 1).astype(np.int64)
    mn = sc * qstar
    out = np.zeros((nblk, bb), np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
    out[:, 2:4] = out[:, 0:2]
    out[:, 4:16] = _scale_bytes(sc.astype(np.uint8), mn.astype(np.uint8))
    lo = np.repeat(qstar[:, 0::2], 32, axis=1)  # units 2g: low nibbles of bytes 32g..
    hi = np.repeat(qstar[:, 1::2], 32, axis=1)
    qs = ((lo & 15) | ((hi & 15) << 4)).astype(np.uint8)
    if ggml_type == Q4:
        out[:, 16:144] = qs
    else:
        # qh[i] bit 2g: +16 for unit 2g's element i; bit 2g + 1: unit 2g + 1's
        qh = np.zeros((nblk, 32), np.int64)
        for g in range(4):
            qh |= ((qstar[:, 2 * g] >> 4) << (2 * g))[:, None]
            qh |= ((qstar[:, 2 * g + 1] >> 4) << (2 * g + 1))[:, None]
        out[:, 16:48] = qh.astype(np.uint8)
        out[:, 48:176] = qs
    kind = (np.arange(nblk) // nb) % ROW_KINDS
    qoff = 16 if ggml_type == Q4 else 48
    for k, frac in FLIP.items():
        if frac == 0.0:
            continue
        sel = kind == k
        flip = (rng.random((nblk, 128)) < frac) & sel[:, None]
        rand = rng.integers(0, 256, (nblk, 128), dtype=np.uint8)
        out[:, qoff:qoff + 128] = np.where(flip, rand, out[:, qoff:qoff + 128])
        if ggml_type == Q5:
            flip_h = (rng.random((nblk, 32)) < frac) & sel[:, None]
            rand_h = rng.integers(0, 256, (nblk, 32), dtype=np.uint8)
            out[:, 16:48] = np.where(flip_h, rand_h, out[:, 16:48])
    normal = np.frombuffer(si_hip.synth_matrix(ggml_type, seed=seed, rows=rows, cols=cols,
                                               threads=8).tobytes(), np.uint8)
    normal = normal.reshape(nblk, bb)
    out = np.where((kind == 3)[:, None], normal, out)
    return out.tobytes()


def row_kinds(rows: int) -> np.ndarray:
    return np.arange(rows) % ROW_KINDS
