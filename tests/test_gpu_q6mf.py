"""GPU parity of several Q6_K columns on the int8 matrix cores
(flh_dot_q6mf.hip: one v_mfma_i32_32x32x16_i8 per 16-weight sub-block of a
32-row tile, the scale products and the fold per lane).

Bar: bitwise against the oracle (fl_dot_i8k_q6_K per column,
src/runtime/quants.h:563-594) and against the streaming kernel
(FLH_NO_Q6MF=1), the routing's size floor lowered (FLH_Q6MF_MIN) so that
small shapes reach the kernel, with old y and padded output strides: 2-8 columns (one
launch; 4-column and 8-column capacity), 9-16 (two), partial last tiles
(rows not a multiple of 32, fewer rows than one tile), 1 to 64 superblocks
per row (both ring depths), the expert-slot form.
"""
import numpy as np
import pytest

from oracle import Q6_K, row_bytes
from util import sane_rows, activations, tuned
from test_gpu_parity import run_dot, bits, say

pytestmark = pytest.mark.gpu

CASES = [(4096, 4096, 2), (4096, 4096, 4), (4096, 4096, 8), (14336, 4096, 3), (4096, 14336, 2), (4096, 14336, 8),
         (33, 256, 5), (31, 1024, 2), (1, 4096, 6), (1000, 8192, 7), (777, 16384, 4), (64, 2816, 8),
         (2049, 1280, 16), (300, 4096, 12), (32, 512, 9)]


@pytest.mark.parametrize("rows,cols,nx", CASES)
def test_q6mf_bitwise(flh, orc, gpu, rows, cols, nx):
    say("q6mf", rows, cols, nx)
    rng = np.random.default_rng(rows * 3 + cols + nx)
    w = sane_rows(Q6_K, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    y0 = rng.standard_normal((nx - 1) * (rows + 2) + rows).astype(np.float32)
    with tuned(flh, FLH_Q6MF_MIN="1,2"):
        got, want = run_dot(flh, orc, gpu, Q6_K, w, rows, cols, xs, ystride=rows + 2, y0=y0)
    assert np.array_equal(bits(got), bits(want))
    with tuned(flh, FLH_NO_Q6MF=1):
        got2, _ = run_dot(flh, orc, gpu, Q6_K, w, rows, cols, xs, ystride=rows + 2, y0=y0)
    assert np.array_equal(bits(got2), bits(got))


def test_q6mf_expert_slot(flh, orc, gpu):
    """STREAM_DOT_IDX: the matrix is expert 2 of 3, the id read on the device."""
    say("q6mf idx")
    rng = np.random.default_rng(5)
    rows, cols, nx = 500, 2048, 4
    rb = rows * row_bytes(Q6_K, cols)
    w = np.concatenate([sane_rows(Q6_K, rows, cols, rng) for _ in range(3)])
    xs = activations(nx, cols, rng, outliers=True)
    with tuned(flh, FLH_Q6MF_MIN="1,2"):
        got, want = run_dot(flh, orc, gpu, Q6_K, w, rows, cols, xs, id_slot=2, estride=rb)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("rows,nx", [(65600, 5), (65600, 8), (65600, 11), (65600, 16), (50000, 9), (14336, 8),
                                     (12300, 6), (14336, 13)])
def test_q6mf_default_routing(flh, orc, gpu, rows, nx):
    """Past the routing floor (12288 rows, 5 columns) with the default tuning:
    a wave per tile (vocab height; 9-16 columns in one pass of six waves per
    workgroup) and four waves per tile (fewer tiles than waves on the chip;
    9-16 columns as two passes), bitwise against the oracle and the streaming
    kernel."""
    cols = 512
    say("q6mf routed", rows, cols, nx)
    rng = np.random.default_rng(nx)
    w = sane_rows(Q6_K, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    got, want = run_dot(flh, orc, gpu, Q6_K, w, rows, cols, xs)
    assert np.array_equal(bits(got), bits(want))
    with tuned(flh, FLH_NO_Q6MF=1):
        got2, _ = run_dot(flh, orc, gpu, Q6_K, w, rows, cols, xs)
    assert np.array_equal(bits(got2), bits(got))
