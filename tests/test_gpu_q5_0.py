"""Q5_0 on the GPU: bit-exact dequant and every STREAM_DOT routing mode.

Q5_0 (22-byte blocks of 32 weights, src/runtime/quants.h:24) is in the
reference's default int8 masks for both engines (src/runtime/kernels.h:
920-930): with int8_dots it takes the q8_1 path fl_dot_i8_q5_0
(quants.h:449-466); otherwise the fast fp32 order over 256-element dequant
chunks (kernels.h:244-254; a row of 1408 columns ends on a half chunk) or the
canonical chain (quants.h:144-162).  Every output must equal the oracle bit
for bit, and the reference's own golden vectors through the device path.
"""
import numpy as np
import pytest

from oracle import Q5_0, row_bytes
from util import sane_rows, activations
from test_gpu_parity import run_dot, bits, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cols", [32, 1408, 4096])
def test_q5_0_dequant_bitexact(flh, orc, gpu, cols):
    say("q5_0 dequant", cols)
    rng = np.random.default_rng(cols + 5)
    rows = 9
    w = sane_rows(Q5_0, rows, cols, rng)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    out = flh.DeviceBuffer(rows * cols * 4)
    flh.dequant(Q5_0, dw, rows, cols, out, gpu)
    got = out.download(np.float32, rows * cols, gpu)
    assert np.array_equal(bits(got), bits(orc.dequant(Q5_0, w, rows, cols).ravel()))


def test_q5_0_golden_vectors(flh, gpu, golden):
    """The reference's own Q5_0 dequant and dot outputs, through the device path."""
    w = golden["dq5_w"]
    dw = flh.DeviceBuffer.from_array(w, gpu)
    out = flh.DeviceBuffer(3 * 1408 * 4)
    flh.dequant(Q5_0, dw, 3, 1408, out, gpu)
    assert np.array_equal(bits(out.download(np.float32, 3 * 1408, gpu)), bits(golden["dq5_out"].ravel()))
    n = int(golden["q5dot_count"][0])
    for i in range(n):
        fmt, cols, rows, nx, st, fast, i8, i8k = (int(v) for v in golden[f"q5dot{i}_meta"])
        say("q5_0 golden dot", i, cols, nx, fast, i8)
        dx = flh.DeviceBuffer.from_array(golden[f"q5dot{i}_x"], gpu)
        dw = flh.DeviceBuffer.from_array(golden[f"q5dot{i}_w"], gpu)
        dy = flh.DeviceBuffer.from_array(golden[f"q5dot{i}_y0"], gpu)
        flh.stream_dot(fmt, dw, rows, cols, dx, dy, gpu, nx=nx, xstride=st, ystride=rows,
                       fast=fast, i8_mask=i8, i8k_mask=i8k)
        assert np.array_equal(bits(dy.download(np.float32, nx * rows, gpu)), bits(golden[f"q5dot{i}_y"])), i


@pytest.mark.parametrize("rows,cols", [(1, 32), (3, 96), (37, 1408), (64, 2048), (17, 4096),
                                       (9, 14336), (5, 16384), (300, 4096)])
def test_q5_0_int8_dot_bitwise(flh, orc, gpu, rows, cols):
    say("q5_0 int8", rows, cols)
    rng = np.random.default_rng(rows * 13 + cols)
    w = sane_rows(Q5_0, rows, cols, rng)
    xs = activations(1, cols, rng, outliers=True)
    y0 = rng.standard_normal(rows).astype(np.float32)
    got, want = run_dot(flh, orc, gpu, Q5_0, w, rows, cols, xs, y0=y0)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("nx", [2, 3, 4, 5, 8])
def test_q5_0_multicol_bitwise(flh, orc, gpu, nx):
    say("q5_0 multicol", nx)
    rng = np.random.default_rng(nx + 77)
    rows, cols = 45, 1408
    w = sane_rows(Q5_0, rows, cols, rng)
    xs = activations(nx, cols, rng)
    got, want = run_dot(flh, orc, gpu, Q5_0, w, rows, cols, xs, ystride=rows + 3,
                        y0=np.zeros((nx - 1) * (rows + 3) + rows, dtype=np.float32))
    assert np.array_equal(bits(got), bits(want))


def test_q5_0_idx_dot(flh, orc, gpu):
    say("q5_0 idx")
    rng = np.random.default_rng(5050)
    rows, cols, ne = 21, 1024, 4
    w = sane_rows(Q5_0, rows * ne, cols, rng)
    xs = activations(1, cols, rng)
    got, want = run_dot(flh, orc, gpu, Q5_0, w, rows, cols, xs, id_slot=2,
                        estride=rows * row_bytes(Q5_0, cols))
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("mode", ["f32fast", "canon"])
@pytest.mark.parametrize("cols", [1408, 4096])
def test_q5_0_fp32_modes_bitwise(flh, orc, gpu, mode, cols):
    say("q5_0 fp32", mode, cols)
    rng = np.random.default_rng(cols + (mode == "canon"))
    rows = 19
    w = sane_rows(Q5_0, rows, cols, rng)
    xs = activations(2, cols, rng)
    got, want = run_dot(flh, orc, gpu, Q5_0, w, rows, cols, xs, mode=mode)
    assert np.array_equal(bits(got), bits(want))
