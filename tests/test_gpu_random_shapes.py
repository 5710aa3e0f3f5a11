"""Randomised shapes through every dot entry point, bitwise against the oracle.

A fixed, seeded list of cases (the same every run): format, rows (1 to ~6000,
log-uniform), columns (multiples of the format's block up to 16384), 1-16
activation columns, output strides with padding, non-zero old y, and the
int8 / q8_1-only / fp32 modes, through flh_stream_dot, flh_act_q8_stream_dot
and the STREAM_DOT_IDX form.  Each case picks its kernel by the library's
own plan, so the list reaches the shapes between the named ones: partial
chunks and tiles, odd superblock counts, workgroups with one row, several
batches.  Bar: every output bit equals the oracle's (fl_dot_i8_q8_0,
fl_dot_i8k_q4_K / _q6_K and the fp32 orders, src/runtime/quants.h:132-642).
"""
import numpy as np
import pytest

from oracle import Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS, col_stride_floats, row_bytes
from util import sane_rows, activations
from test_gpu_parity import run_dot, bits, say, dev_cols

pytestmark = pytest.mark.gpu

BLOCK = {Q8_0: 32, Q5_0: 32, Q4_K: 256, Q6_K: 256, IQ2_XXS: 256, IQ3_XXS: 256}


def make_cases(n=72, seed=2026):
    rng = np.random.default_rng(seed)
    fmts = [Q4_K, Q4_K, Q4_K, Q6_K, Q6_K, Q8_0, Q8_0, Q5_0, IQ2_XXS, IQ3_XXS]
    cases = []
    for i in range(n):
        fmt = fmts[rng.integers(len(fmts))]
        rows = int(np.exp(rng.uniform(0, np.log(6000))))
        nblk = int(rng.integers(1, 16384 // BLOCK[fmt] + 1))
        if fmt in (IQ2_XXS, IQ3_XXS):
            nblk = max(1, nblk // 8) * 8 if rng.random() < 0.5 else nblk
        cols = nblk * BLOCK[fmt]
        while rows * cols > 24_000_000:
            rows = max(1, rows // 2)
        nx = 1 if rng.random() < 0.4 else int(rng.integers(2, 17))
        mode = "int8"
        r = rng.random()
        if fmt in (IQ2_XXS, IQ3_XXS):
            mode = "iq8" if r < 0.8 else "f32fast"
        elif r < 0.1:
            mode = "f32fast"
        elif r < 0.15:
            mode = "canon"
        elif r < 0.25 and fmt in (Q4_K, Q6_K):
            mode = "q81"
        pad = int(rng.integers(0, 4))
        kind = "dot"
        if nx == 1 and fmt in (Q4_K, Q6_K) and mode == "int8" and rng.random() < 0.4:
            kind = "fused"
        elif rng.random() < 0.1:
            kind = "idx"
        cases.append((i, fmt, rows, cols, nx, mode, pad, kind))
    return cases


CASES = make_cases()


@pytest.mark.parametrize("i,fmt,rows,cols,nx,mode,pad,kind", CASES)
def test_random_shape_bitwise(flh, orc, gpu, i, fmt, rows, cols, nx, mode, pad, kind):
    say("random", i, fmt, rows, cols, nx, mode, pad, kind)
    rng = np.random.default_rng(1000 + i)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    ys = rows + pad
    y0 = rng.standard_normal((nx - 1) * ys + rows).astype(np.float32)
    if kind == "fused":
        st = col_stride_floats(cols)
        dx, _ = dev_cols(flh, gpu, xs, st)
        dy = flh.DeviceBuffer.from_array(y0, gpu)
        dw = flh.DeviceBuffer.from_array(w, gpu)
        flh.act_q8_stream_dot(fmt, dw, rows, cols, dx, dy, gpu)
        got = dy.download(np.float32, y0.size, gpu)
        want = y0.copy()
        orc.stream_dot(fmt, w, rows, cols, orc.act_q8_cols(xs, st), want, threads=8)
    elif kind == "idx":
        # the matrix is expert 2 of 3 (the others random bytes): the id is read on the device
        e = 2
        rb = rows * row_bytes(fmt, cols)
        ww = np.concatenate([sane_rows(fmt, rows, cols, rng), sane_rows(fmt, rows, cols, rng), w])
        got, want = run_dot(flh, orc, gpu, fmt, ww, rows, cols, xs, mode=mode, y0=y0, id_slot=e,
                            estride=rb, ystride=ys)
    else:
        got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode=mode, y0=y0, ystride=ys)
    assert np.array_equal(bits(got), bits(want))
