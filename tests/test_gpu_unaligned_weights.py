"""Weights at a 2-byte (not 4-byte) aligned address, bitwise against the oracle.

The 2-byte aligned block formats (Q8_0 34 B, Q5_0 22 B, Q6_K 210 B,
IQ2_XXS 66 B, IQ3_XXS 98 B) put a row tile at an address 2 mod 4 whenever a
row is 2 mod 4 bytes long (Q6_K with an odd number of superblocks per row,
e.g. 11008 columns; Q8_0 / Q5_0 with cols % 64 == 32), which the reference's
graph builder does when it splits a matrix into row tiles
(src/model/decoder.cpp:482-528) and which STREAM_DOT_IDX does with such an
expert stride.  The kernels that need 16-byte aligned weights decline those
and the register / fp32 kernels read them through aligned windows; every
mode must give the oracle's bits (fl_dot_i8_q8_0, fl_dot_i8k_q6_K and the
fp32 orders, src/runtime/quants.h:132-642)."""
import numpy as np
import pytest

from oracle import Q8_0, Q5_0, Q6_K, IQ2_XXS, IQ3_XXS, Q4_K, col_stride_floats, row_bytes
from util import sane_rows, activations
from test_gpu_parity import bits, say, dev_cols, I8, I8K

pytestmark = pytest.mark.gpu

MODES = {"int8": (1, I8, I8K), "q81": (1, I8, 0), "f32fast": (1, 0, 0), "canon": (0, 0, 0),
         "iq8": (1, 0b1100000, 0)}


def run(flh, orc, gpu, fmt, rows, cols, nx, mode, off, seed, idx=False):
    rng = np.random.default_rng(seed)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    st = col_stride_floats(cols)
    fast, i8, i8k = MODES[mode]
    dx, _ = dev_cols(flh, gpu, xs, st)
    flh.act_q8(dx, cols, gpu, nx=nx, xstride=st)
    ref_x = orc.act_q8_cols(xs, st)
    y0 = rng.standard_normal((nx - 1) * rows + rows).astype(np.float32)
    dy = flh.DeviceBuffer.from_array(y0, gpu)
    want = y0.copy()
    if idx:
        # expert 1 of 2 at stride rows * row_bytes (2 mod 4 here), the base at off
        rb = rows * row_bytes(fmt, cols)
        other = sane_rows(fmt, rows, cols, rng)
        dw = flh.DeviceBuffer.from_array(np.concatenate([np.zeros(off, np.uint8), other, w]), gpu)
        slot = flh.DeviceBuffer.from_array(np.array([1], dtype=np.uint32), gpu)
        flh.stream_dot(fmt, dw.ptr + off, rows, cols, dx, dy, gpu, nx=nx, xstride=st, ystride=rows,
                       id_slot=slot, estride=rb, fast=fast, i8_mask=i8, i8k_mask=i8k)
    else:
        dw = flh.DeviceBuffer.from_array(np.concatenate([np.zeros(off, np.uint8), w]), gpu)
        flh.stream_dot(fmt, dw.ptr + off, rows, cols, dx, dy, gpu, nx=nx, xstride=st, ystride=rows,
                       fast=fast, i8_mask=i8, i8k_mask=i8k)
    orc.stream_dot(fmt, w, rows, cols, ref_x, want, nx=nx, xstride=st, ystride=rows, fast=fast,
                   i8_mask=i8, i8k_mask=i8k, threads=8)
    got = dy.download(np.float32, y0.size, gpu)
    assert np.array_equal(bits(got), bits(want))


CASES = [
    (Q6_K, 301, 11008, 1), (Q6_K, 300, 11008, 3), (Q6_K, 1000, 2816, 1), (Q6_K, 77, 768, 16),
    (Q8_0, 333, 4064, 1), (Q8_0, 300, 4096, 2), (Q8_0, 65, 14336, 8),
    (Q5_0, 333, 4064, 1), (Q5_0, 200, 1056, 4),
    (IQ2_XXS, 129, 4096, 1), (IQ3_XXS, 129, 2304, 3),
]


@pytest.mark.parametrize("fmt,rows,cols,nx", CASES)
def test_two_byte_aligned_weights(flh, orc, gpu, fmt, rows, cols, nx):
    iq = fmt in (IQ2_XXS, IQ3_XXS)
    for mode in (("iq8", "f32fast", "canon") if iq else ("int8", "q81", "f32fast", "canon")):
        if mode == "q81" and fmt != Q6_K:
            continue
        say("unaligned w", fmt, rows, cols, nx, mode)
        run(flh, orc, gpu, fmt, rows, cols, nx, mode, 2, rows + cols + nx)


@pytest.mark.parametrize("fmt,rows,cols", [(Q6_K, 301, 11008), (Q8_0, 333, 4064), (Q5_0, 333, 4064),
                                           (IQ2_XXS, 129, 2304)])
def test_two_byte_aligned_expert_stride(flh, orc, gpu, fmt, rows, cols):
    """STREAM_DOT_IDX with an expert stride of 2 mod 4 bytes (odd rows of
    2 mod 4-byte rows): expert 1 starts at an address 2 mod 4."""
    assert (rows * row_bytes(fmt, cols)) % 4 == 2
    mode = "iq8" if fmt == IQ2_XXS else "int8"
    say("unaligned idx", fmt, rows, cols)
    run(flh, orc, gpu, fmt, rows, cols, 1, mode, 0, 7 * rows + cols, idx=True)


def test_q4_k_and_f32_keep_four_byte_alignment(flh, gpu):
    """Q4_K (144-byte superblocks: an aligned matrix never yields a 2 mod 4
    tile) and F32 weights at an address 2 mod 4 are an argument error."""
    dw = flh.DeviceBuffer(4096)
    dx = flh.DeviceBuffer(64 << 10)
    dy = flh.DeviceBuffer(4096)
    for fmt in (Q4_K, 0):
        with pytest.raises(flh.FlhError):
            flh.stream_dot(fmt, dw.ptr + 2, 1, 256, dx, dy, gpu)
