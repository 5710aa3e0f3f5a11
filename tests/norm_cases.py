"""Seeded inputs of the RMSNORM golden cases (tests/golden/make_norm_golden.py
writes the reference's outputs for them; the tests regenerate the inputs
from the seeds and check their digest before comparing outputs).

NORM_CASES: (n, seed, outlier_scale) -- x N(0,1) with 1 % of the entries
scaled by outlier_scale, norm weight 1 + 0.1 N(0,1), eps 1e-5.
CHAIN_CASES: (rows, cols, seed) -- the decoder's norm -> quant -> matvec
chain (src/model/decoder.cpp:874-880) into a Q4_K matrix of random blocks
with sane scales, y starting at zero."""
import hashlib

import numpy as np

from oracle import Q4_K
from util import sane_rows

EPS = 1e-5
NORM_CASES = [(256, 201, 20.0), (4096, 202, 20.0), (14336, 203, 20.0), (4096, 204, 1000.0), (1024, 205, 1e-3)]
CHAIN_CASES = [(300, 4096, 211), (200, 14336, 212)]


def norm_inputs(n, seed, outlier_scale):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32)
    x[rng.random(n) < 0.01] *= np.float32(outlier_scale)
    wn = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    return x, wn


def chain_inputs(rows, cols, seed):
    x, wn = norm_inputs(cols, seed, 20.0)
    w = sane_rows(Q4_K, rows, cols, np.random.default_rng(seed + 1000))
    return x, wn, w


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.digest()
