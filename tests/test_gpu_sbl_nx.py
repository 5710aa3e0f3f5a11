"""GPU parity of the several-column superblock-per-lane kernel
(k_dot_sbl_nx, fast-llm_amd/csrc/flh_dot_sbl.hip): 2..8 activation columns of
Q8_0, Q5_0, IQ2_XXS and IQ3_XXS x q8_1 in one pass over the weights.

Bar: bitwise against the oracle's per-column dots (fl_dot_i8_q8_0 /
fl_dot_i8_q5_0, src/runtime/quants.h:438-466; the IQ group order of
kernels_gpu.h:759-852) with y += accumulation onto random y, for every column
count up to the 8-column capacity (idle capacity columns store nothing) and
9..16 columns in two passes, row
geometries with partial last chunks and idle lanes, widths where 8 columns do
not fit (8192: the register kernel takes them), wave counts, grids small
enough that every wave streams many chunks, an expert picked by an id slot,
and against the register kernel (FLH_SBL=0) on a 14336x4096 matrix.
"""
import numpy as np
import pytest

from util import tuned, sane_rows, activations
from test_gpu_parity import bits, say, run_dot

pytestmark = pytest.mark.gpu

Q8_0, Q5_0, IQ2_XXS, IQ3_XXS = 1, 2, 5, 6
MODE = {Q8_0: "int8", Q5_0: "int8", IQ2_XXS: "iq8", IQ3_XXS: "iq8"}
FMTS = [Q8_0, Q5_0, IQ2_XXS, IQ3_XXS]
# (rows, cols): 4, 8, 16, 32 lanes per row (IQ rows need whole superblock pairs)
SHAPES = [(33, 1024), (13, 2048), (1001, 4096), (70, 8192)]


def case(flh, orc, gpu, fmt, rows, cols, nx, seed, cfg="1"):
    rng = np.random.default_rng(seed)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    y0 = rng.standard_normal(nx * rows).astype(np.float32)
    with tuned(flh, FLH_SBL=cfg):
        got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode=MODE[fmt], y0=y0)
    assert np.array_equal(bits(got), bits(want))
    return got


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("nx", [2, 3, 4, 5, 8])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_sbl_nx_bitwise(flh, orc, gpu, fmt, nx, rows, cols):
    say("sbl nx", fmt, nx, rows, cols)
    case(flh, orc, gpu, fmt, rows, cols, nx, rows * 13 + cols + 7 * nx + fmt)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("nx", [9, 12, 16])
@pytest.mark.parametrize("rows,cols", [(1001, 4096), (70, 8192)])
def test_sbl_nx_two_passes(flh, orc, gpu, fmt, nx, rows, cols):
    """9..16 columns: two passes (8 + the rest, 7 + 2 for 9); at 8192 columns
    the 8-column pass does not fit and the whole tile takes the register
    kernel (no column is added twice)."""
    say("sbl nx passes", fmt, nx, rows, cols)
    case(flh, orc, gpu, fmt, rows, cols, nx, rows + cols + 17 * nx + fmt)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("cfg", ["1,8,1,0", "1,4,2,0,255", "1,4,1,3,1", "1,8,1,5,2"])
def test_sbl_nx_launch_shapes(flh, orc, gpu, fmt, cfg):
    """8-wave workgroups, two workgroups per CU, 3 or 5 workgroups in all
    (dozens of chunks per wave), 1-255 waves requesting weights early."""
    say("sbl nx cfg", fmt, cfg)
    case(flh, orc, gpu, fmt, 777, 4096, 6, 31 + fmt, cfg)


@pytest.mark.parametrize("fmt", FMTS)
def test_sbl_nx_matches_register_kernel(flh, orc, gpu, fmt):
    """The several-column kernel and the register kernel give the same bits
    (and the oracle's) at 14336x4096 with 8 columns; an id slot picks the
    expert."""
    say("sbl nx vs register", fmt)
    rows, cols, nx = 14336, 4096, 8
    outs = [case(flh, orc, gpu, fmt, rows, cols, nx, 500 + fmt, cfg) for cfg in ("1", "0")]
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
    rng = np.random.default_rng(600 + fmt)
    r, ne = 96, 3
    we = sane_rows(fmt, r * ne, cols, rng)
    xs = activations(4, cols, rng, outliers=True)
    got, want = run_dot(flh, orc, gpu, fmt, we, r, cols, xs, mode=MODE[fmt], id_slot=2,
                        estride=r * flh.row_bytes(fmt, cols))
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("env", [{"FLH_SBL_NX_DEP": "2"}, {"FLH_SBL": "1,8", "FLH_SBL_NX_DEP": "2"},
                                 {"FLH_SBL": "1,8", "FLH_SBL_NX_DEP": "1"}])
def test_sbl_nx_ring_depth_keeps_bits(flh, orc, gpu, fmt, env):
    """FLH_SBL_NX_DEP: 2-stage rings (4 waves, or 8 where they fit) give the
    planned 1-stage run's bits, and the oracle's."""
    say("sbl nx ring depth", fmt, env)
    rows, cols, nx = 1001, 4096, 5
    base = case(flh, orc, gpu, fmt, rows, cols, nx, 77 + fmt)
    rng = np.random.default_rng(77 + fmt)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    y0 = rng.standard_normal(nx * rows).astype(np.float32)
    with tuned(flh, **env):
        got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode=MODE[fmt], y0=y0)
    assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(bits(got), bits(base))
