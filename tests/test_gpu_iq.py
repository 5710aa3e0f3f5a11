"""IQ2_XXS / IQ3_XXS on the GPU, bitwise against the oracle.

The reference runs codebook formats on its CPU only through the canonical
chain (fl_dot_row_iq2_xxs / fl_dot_row_iq3_xxs, src/runtime/quants.h:237-290;
golden vectors from its own code here), and on its GPU through q8_1 int8
kernels (src/runtime/kernels_gpu.h:759-852, default GPU mask kernels.h:928-
930).  Device dequant, canonical, fast-fp32 and q8_1 int8 outputs must each
equal the oracle bit for bit, and the canonical ones the reference's own.
"""
import numpy as np
import pytest

from oracle import IQ2_XXS, IQ3_XXS, row_bytes
from util import sane_rows, activations
from test_gpu_parity import run_dot, bits, say

pytestmark = pytest.mark.gpu
FMTS = [IQ2_XXS, IQ3_XXS]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("cols", [256, 4096])
def test_iq_dequant_bitexact(flh, orc, gpu, fmt, cols):
    say("iq dequant", fmt, cols)
    rng = np.random.default_rng(cols + fmt)
    rows = 11
    w = sane_rows(fmt, rows, cols, rng)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    out = flh.DeviceBuffer(rows * cols * 4)
    flh.dequant(fmt, dw, rows, cols, out, gpu)
    got = out.download(np.float32, rows * cols, gpu)
    assert np.array_equal(bits(got), bits(orc.dequant(fmt, w, rows, cols).ravel()))


def test_iq_reference_canonical_vectors(flh, gpu, golden):
    """The reference's own canonical IQ dots and its KAT block, on the device."""
    for i in range(int(golden["iqdot_count"][0])):
        fmt, cols, rows, nx, st, fast, i8, i8k = (int(v) for v in golden[f"iqdot{i}_meta"])
        say("iq golden", i, fmt, cols, nx)
        dx = flh.DeviceBuffer.from_array(golden[f"iqdot{i}_x"], gpu)
        dw = flh.DeviceBuffer.from_array(golden[f"iqdot{i}_w"], gpu)
        dy = flh.DeviceBuffer.from_array(golden[f"iqdot{i}_y0"], gpu)
        flh.stream_dot(fmt, dw, rows, cols, dx, dy, gpu, nx=nx, xstride=st, ystride=rows,
                       fast=False, i8_mask=0, i8k_mask=0)
        assert np.array_equal(bits(dy.download(np.float32, nx * rows, gpu)), bits(golden[f"iqdot{i}_y"])), i
    dw = flh.DeviceBuffer.from_array(golden["iq_kat_w"], gpu)
    dx = flh.DeviceBuffer.from_array(golden["iq_kat_x"], gpu)
    dy = flh.DeviceBuffer(4)
    dy.zero(gpu)
    flh.stream_dot(IQ2_XXS, dw, 1, 256, dx, dy, gpu, fast=False)
    assert dy.download(np.float32, 1, gpu)[0] == golden["iq_kat_y"][0] == 2.0


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 512), (65, 2048), (300, 4096), (9, 14336),
                                       (4, 16384)])
def test_iq_int8_bitwise(flh, orc, gpu, fmt, rows, cols):
    say("iq int8", fmt, rows, cols)
    rng = np.random.default_rng(rows * 31 + cols + fmt)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(1, cols, rng, outliers=True)
    y0 = rng.standard_normal(rows).astype(np.float32)
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode="iq8", y0=y0)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("nx", [2, 3, 4, 8])
def test_iq_int8_multicol(flh, orc, gpu, fmt, nx):
    say("iq multicol", fmt, nx)
    rng = np.random.default_rng(nx * 5 + fmt)
    rows, cols = 37, 4096
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng)
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode="iq8", ystride=rows + 5,
                        y0=np.zeros((nx - 1) * (rows + 5) + rows, dtype=np.float32))
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", FMTS)
def test_iq_int8_idx(flh, orc, gpu, fmt):
    say("iq idx", fmt)
    rng = np.random.default_rng(77 + fmt)
    rows, cols, ne = 24, 2048, 3
    w = sane_rows(fmt, rows * ne, cols, rng)
    xs = activations(1, cols, rng)
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode="iq8", id_slot=2,
                        estride=rows * row_bytes(fmt, cols))
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("mode", ["f32fast", "canon"])
def test_iq_fp32_modes_bitwise(flh, orc, gpu, fmt, mode):
    say("iq fp32", fmt, mode)
    rng = np.random.default_rng(fmt * 3 + (mode == "canon"))
    rows, cols = 21, 2048
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(2, cols, rng)
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode=mode)
    assert np.array_equal(bits(got), bits(want))
