"""GPU parity of several activation columns over wide rows on the streaming
kernel (flh_dot_kstream.hip), whose LDS plan for them holds one workgroup
per CU: Q6_K (5-8 columns in one pass) and Q4_K, with the matrix-core
kernels switched off.

Bar: bitwise against the oracle (fl_dot_i8k_q6_K / fl_dot_i8k_q4_K per
column, src/runtime/quants.h:538-594), with old y and padded output strides:
2-8 columns (one pass), 9-16 (two passes), 256-16384 columns, row counts
that leave a partial last batch.
"""
import numpy as np
import pytest

from oracle import Q4_K, Q6_K
from util import sane_rows, activations, tuned
from test_gpu_parity import run_dot, bits, say

pytestmark = pytest.mark.gpu

CASES = [(Q6_K, 4096, 14336, 2), (Q6_K, 4096, 14336, 4), (Q6_K, 1000, 16384, 3), (Q6_K, 333, 12288, 4),
         (Q6_K, 4096, 14336, 8), (Q6_K, 64, 14336, 2), (Q6_K, 777, 14336, 6),
         (Q4_K, 4096, 14336, 4), (Q4_K, 1001, 16384, 3), (Q4_K, 300, 12288, 7),
         # Q6_K: 5-8 columns in one pass, 9-16 as a pass of 8 and the rest
         (Q6_K, 14336, 4096, 8), (Q6_K, 4096, 4096, 5), (Q6_K, 1000, 2816, 7), (Q6_K, 300, 14336, 8),
         (Q6_K, 4096, 14336, 16), (Q6_K, 77, 256, 6), (Q6_K, 5000, 1024, 12), (Q6_K, 2049, 8192, 13)]


@pytest.mark.parametrize("fmt,rows,cols,nx", CASES)
def test_kstream_wide_rows_bitwise(flh, orc, gpu, fmt, rows, cols, nx):
    say("kstream wide", fmt, rows, cols, nx)
    rng = np.random.default_rng(fmt * 13 + rows + cols + nx)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    y0 = rng.standard_normal((nx - 1) * (rows + 1) + rows).astype(np.float32)
    with tuned(flh, FLH_NO_MFMA=1, FLH_NO_Q6MF=1):
        got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, ystride=rows + 1, y0=y0)
    assert np.array_equal(bits(got), bits(want))
