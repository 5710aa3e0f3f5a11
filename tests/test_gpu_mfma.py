"""GPU parity of the multi-column Q4_K kernel on the int8 matrix cores
(flh_dot_mfma.hip, used by STREAM_DOT for 2..16 Q4_K columns).

Bar: bitwise against the oracle (the reference's fl_dot_i8k_q4_K per column,
src/runtime/quants.h:538-561), at the speculative-verify shapes of the
benchmark (14336x4096 and 4096x14336, N in {2, 4, 8}) and at shapes that
exercise partial 16-row tiles, several row batches per workgroup, column
groups (the 14336-column plan holds 4 columns), the 16-column maximum, and
one 16-row tile per workgroup with 5-8 columns of 48-64 superblocks, where each
chunk's DMA carries its own activation blocks (4096x14336 N=8, 250x14336 N=7,
100x12288 N=6, 40x16384 N=5).
"""
import os

import numpy as np
import pytest

from oracle import Q4_K
from util import sane_rows, activations, tuned
from test_gpu_parity import run_dot, bits, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols,nx", [
    (14336, 4096, 2), (14336, 4096, 4), (14336, 4096, 8),
    (4096, 14336, 2), (4096, 14336, 4), (4096, 14336, 8),
    (20000, 512, 16), (300, 4096, 3), (17, 256, 2), (4100, 2048, 7), (40, 16384, 5),
    (4096, 14336, 13), (100, 12288, 6), (250, 14336, 7),
])
def test_mfma_multicol_bitwise(flh, orc, gpu, rows, cols, nx):
    say("mfma", rows, cols, nx)
    rng = np.random.default_rng(rows + 7 * cols + nx)
    w = sane_rows(Q4_K, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    got, want = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs, ystride=rows + 1,
                        y0=rng.standard_normal((nx - 1) * (rows + 1) + rows).astype(np.float32))
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("rows,cols,nx", [
    (20000, 1024, 16), (7777, 2816, 5), (9000, 1280, 3), (12345, 4096, 4), (8200, 1024, 12), (16000, 3328, 8),
])
def test_mfma_register_accumulators_bitwise(flh, orc, gpu, rows, cols, nx):
    """Shapes on the register-accumulator layout (two or more 16-row tiles per
    batch): 16 columns at 4 superblocks per row, accumulator classes of unequal
    length (11, 5, 13 superblocks per row), odd tile counts and partial last
    tiles; bitwise against the oracle and against the parked-term layout."""
    say("mfma own", rows, cols, nx)
    rng = np.random.default_rng(rows + 3 * cols + nx)
    w = sane_rows(Q4_K, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    y0 = rng.standard_normal((nx - 1) * (rows + 2) + rows).astype(np.float32)
    got, want = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs, ystride=rows + 2, y0=y0)
    assert np.array_equal(bits(got), bits(want))
    with tuned(flh, FLH_MFMA_OWN=0):
        got2, _ = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs, ystride=rows + 2, y0=y0)
    assert np.array_equal(bits(got2), bits(got))


@pytest.mark.parametrize("rows,cols,nx", [
    (4096, 14336, 8), (20000, 2304, 8), (1000, 2560, 5), (333, 2816, 16), (4100, 4096, 3), (40, 16384, 7),
])
def test_mfma_k_halves_bitwise(flh, orc, gpu, rows, cols, nx):
    """K halves forced (superblocks split by sb % 4 into two staged halves):
    odd superblock counts, several row batches (the halves alternate), 16
    columns, partial tiles."""
    say("mfma k-halves", rows, cols, nx)
    rng = np.random.default_rng(rows + 5 * cols + nx)
    w = sane_rows(Q4_K, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    with tuned(flh, FLH_MFMA_TUNE="2,0,1"):
        got, want = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs, ystride=rows + 3,
                            y0=rng.standard_normal((nx - 1) * (rows + 3) + rows).astype(np.float32))
    assert np.array_equal(bits(got), bits(want))


def test_mfma_equals_streaming_kernel(flh, orc, gpu):
    """Same bits with the matrix-core kernel switched off (streaming kernel)."""
    say("mfma vs kstream")
    rng = np.random.default_rng(3)
    rows, cols, nx = 1000, 4096, 4
    plan = flh.mfma_plan(rows, cols, nx)
    assert not plan["xc"] and not plan["kh"], plan          # the activations fit whole
    w = sane_rows(Q4_K, rows, cols, rng)
    xs = activations(nx, cols, rng)
    got, want = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs)
    with tuned(flh, FLH_NO_MFMA=1):
        got2, _ = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs)
    assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(bits(got2), bits(got))


@pytest.mark.parametrize("rows,cols,nx", [(4096, 14336, 8), (250, 14336, 7)])
def test_mfma_activations_in_chunk_equals_k_halves(flh, orc, gpu, rows, cols, nx):
    """One 16-row tile per workgroup with activations too wide to stage
    whole: the activations-in-chunk mode (default) and K halves (FLH_MFMA_XC=0)
    give the same bits, and both equal the oracle.  The plan query confirms
    which mode each run took."""
    say("mfma xc vs kh", rows, cols, nx)
    plan = flh.mfma_plan(rows, cols, nx)
    assert plan["xc"] and not plan["kh"] and plan["nrb"] == 16, plan
    rng = np.random.default_rng(rows + 11 * cols + nx)
    w = sane_rows(Q4_K, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    y0 = rng.standard_normal((nx - 1) * rows + rows).astype(np.float32)
    got, want = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs, y0=y0)
    with tuned(flh, FLH_MFMA_XC=0):
        plan = flh.mfma_plan(rows, cols, nx)
        assert plan["kh"] and not plan["xc"], plan
        got2, _ = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs, y0=y0)
    assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(bits(got2), bits(got))
