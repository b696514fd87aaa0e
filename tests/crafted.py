"""Crafted weights and activations that stress the matrix-core kernels'
fixed-point activations (test infrastructure).

The kernels write each 256-element block of x as X * 2^(e - 30), e from the
block's largest |x|.  An activation far below that maximum keeps few
significant bits, so the inputs here put one large activation in every
16-element chunk on a weight that is exactly zero (the dot does not see it)
and small activations everywhere else, which then carry the whole dot:

  "tiny"  x = +-1 on the zero weights, +-(0.5..2)e-7 elsewhere
  "side"  x = +-1 on the zero weights, 1..8 elements of +-(0.5..2)e-6 per
          block (as many as a block's side list holds), the rest 0
  "edge"  x = +-1 on the zero weights, +-2^-13 (1..1.5) elsewhere: just above
          the side threshold 2^(e - 14) of a block whose maximum is 1 (e = 1)
  "many"  x = +-1 next to the zero weights (element 16 c + 1), 9..16 elements
          of +-(0.5..2)e-6 per block, the rest 0: more side elements than a
          block lists, on a dot that the large activations carry

Zero weights: Q4_K q = 0 with every min 0; Q5_K q = 0 (qh bit clear) with
every min 0; Q6_K q = 32 (quant.rs:36-63, 90-122, 145-171).
"""
from __future__ import annotations

import numpy as np

import si_hip

BLOCK = {12: 144, 13: 176, 14: 210}
ZERO_ELEMS = np.arange(0, 256, 16)  # element 16 c of every chunk c
CASES = ("tiny", "side", "edge", "many")


def _set_nibble(a, byte, hi, value):
    if hi:
        a[:, byte] = (a[:, byte] & 0x0F) | (value << 4)
    else:
        a[:, byte] = (a[:, byte] & 0xF0) | value


def zero_weight_matrix(t: int, rows: int, cols: int, seed: int, zero_elems=ZERO_ELEMS):
    """Synthetic matrix of type t whose weights at `zero_elems` of every block
    are exactly 0 (Q4_K/Q5_K: every min is 0 as well)."""
    w = np.array(si_hip.synth_matrix(t, seed=seed, rows=rows, cols=cols, threads=8), np.uint8)
    a = w.reshape(-1, BLOCK[t])
    if t in (12, 13):
        a[:, 8:12] = 0        # scales bytes 4..7: mins of units 0..3, high bits of 4..7
        a[:, 12:16] &= 0x0F   # scales bytes 8..11: high nibble = low bits of mins 4..7
    for i in zero_elems:
        i = int(i)
        if t == 14:
            h, t4, l = i // 128, (i % 128) // 32, i % 32
            _set_nibble(a, 64 * h + l + 32 * (t4 & 1), t4 >> 1, 0)
            qh = 128 + 32 * h + l
            a[:, qh] = (a[:, qh] & ~np.uint8(3 << (2 * t4))) | np.uint8(2 << (2 * t4))
        else:
            u, l = i // 32, i % 32
            qs = (16 if t == 12 else 48) + 32 * (u // 2) + l
            _set_nibble(a, qs, u & 1, 0)
            if t == 13:
                a[:, 16 + l] &= ~np.uint8(1 << u)
    return w


def crafted_x(cols: int, case: str, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    nb = cols // 256
    x = np.zeros((nb, 256), np.float64)
    sign = lambda shape: rng.choice([-1.0, 1.0], size=shape)
    x[:, ZERO_ELEMS] = sign((nb, len(ZERO_ELEMS)))
    others = np.setdiff1d(np.arange(256), ZERO_ELEMS)
    if case == "tiny":
        x[:, others] = sign((nb, others.size)) * rng.uniform(0.5e-7, 2e-7, (nb, others.size))
    elif case == "side":
        for b in range(nb):
            k = 1 + b % 8
            pos = rng.choice(others, size=k, replace=False)
            x[b, pos] = sign(k) * rng.uniform(0.5e-6, 2e-6, k)
    elif case == "edge":
        x[:, others] = sign((nb, others.size)) * 2.0 ** -13 * rng.uniform(1.0, 1.5,
                                                                         (nb, others.size))
    elif case == "many":
        x[:, ZERO_ELEMS] = 0.0
        x[:, ZERO_ELEMS + 1] = sign((nb, len(ZERO_ELEMS)))
        rest = np.setdiff1d(others, ZERO_ELEMS + 1)
        for b in range(nb):
            k = 9 + b % 8
            pos = rng.choice(rest, size=k, replace=False)
            x[b, pos] = sign(k) * rng.uniform(0.5e-6, 2e-6, k)
    else:
        raise ValueError(case)
    return x.reshape(-1).astype(np.float32)
