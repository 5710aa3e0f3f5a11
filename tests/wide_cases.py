"""Seeded inputs of the wide golden cases (tests/golden/make_wide_golden.py
writes the reference's outputs for them; the GPU tests regenerate the same
bytes and check them against the stored digest before comparing outputs)."""
import hashlib

import numpy as np

from oracle import Q8_0, Q4_K, Q6_K
from util import sane_rows

# (fmt, rows, cols, nx, seed): the Llama-3-8B widths of BASELINE configs 1-4
WIDE_CASES = [
    (Q4_K, 300, 4096, 1, 101), (Q4_K, 300, 4096, 2, 102), (Q4_K, 300, 4096, 4, 103), (Q4_K, 300, 4096, 8, 104),
    (Q4_K, 200, 14336, 1, 105), (Q4_K, 200, 14336, 2, 106), (Q4_K, 200, 14336, 4, 107), (Q4_K, 200, 14336, 8, 108),
    (Q6_K, 300, 4096, 1, 109), (Q6_K, 200, 14336, 1, 110), (Q8_0, 300, 4096, 1, 111),
]
# Q8_0 weight quantizer fixture: rows, cols, seed of N(0, 0.02^2) floats
Q8_0_QUANT = (16, 4096, 112)


def wide_case_inputs(fmt, rows, cols, nx, seed):
    """Weights (random blocks with sane scales), nx activation columns
    (N(0,1), 1 % x20 outliers) and the initial y, all from one seed."""
    rng = np.random.default_rng(seed)
    w = sane_rows(fmt, rows, cols, rng)
    xs = rng.standard_normal((nx, cols)).astype(np.float32)
    m = rng.random(size=xs.shape) < 0.01
    xs[m] *= 20.0
    y0 = rng.standard_normal(nx * rows).astype(np.float32)
    return w, xs, y0


def digest(w, xs, y0):
    h = hashlib.sha256()
    for a in (w, xs, y0):
        h.update(np.ascontiguousarray(a).tobytes())
    return h.digest()
