"""GPU parity of the fast fp32 order of the 256-element chunk formats (Q4_K,
Q6_K, Q5_0, IQ2_XXS, IQ3_XXS: k_dot_fastk in flh_f32.hip; the reference's
dot_row_fast_dequant, src/runtime/kernels.h:59-104,162-254), the route the
reference's GPU masks give Q6_K and its CPU masks give the IQ formats, and of F32
and Q8_0 weights (k_dot_f32row; dot_row_fast / dot_row_fast_q8_0,
kernels.h:11-19,58-130), the route of every F32 matrix such as an MoE
router.

Bar: bitwise against the oracle.  Seeded random cases cover what the
kernel's plan varies with: rows per wave (1 to 4: up to 70000 rows, with a
partial last workgroup), activation tiles (one tile, several, a last partial
tile; 1 to 16 columns, the 16-column tile of 4 superblocks), rows of 1 to 64
superblocks (partial last pass), output strides with padding, old y, and the
expert-slot form (STREAM_DOT_IDX: the matrix is expert 2 of 3, the id read on
the device).
"""
import numpy as np
import pytest

from oracle import F32, Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS, row_bytes, col_stride_floats
from util import sane_rows, activations, normal_weights
from test_gpu_parity import run_dot, bits, say, dev_cols, I8, I8K

pytestmark = pytest.mark.gpu


def make_cases(n=48, seed=77):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        fmt = (Q4_K, Q6_K, Q4_K, Q6_K, Q5_0, IQ2_XXS, IQ3_XXS)[rng.integers(7)]
        rows = int(np.exp(rng.uniform(0, np.log(70000))))
        nsb = int(rng.integers(1, 65))
        nx = 1 if rng.random() < 0.5 else int(rng.integers(2, 17))
        while rows * nsb * max(1, nx // 4) > 1_200_000:   # the oracle's share stays small
            rows = max(1, rows // 2)
        pad = int(rng.integers(0, 3))
        idx = rng.random() < 0.2
        cols = 256 * nsb
        if fmt == Q5_0 and rng.random() < 0.6:              # a last chunk of 1-7 blocks
            cols = 256 * (nsb - 1) + 32 * int(rng.integers(1, 8))
        cases.append((i, fmt, rows, cols, nx, pad, idx))
    cases += [(105, Q5_0, 300, 32, 1, 0, False), (106, Q5_0, 4096, 14336 + 96, 1, 0, False),
              (107, IQ2_XXS, 4096, 4096, 1, 0, False), (108, IQ3_XXS, 40000, 4096, 2, 1, True),
              (109, Q5_0, 77, 2816, 16, 2, False), (100, Q6_K, 70001, 256, 1, 0, False), (101, Q4_K, 33000, 512, 1, 1, False),
              (102, Q6_K, 40000, 1280, 3, 0, True), (103, Q6_K, 128, 16384, 1, 0, False),
              (104, Q4_K, 37, 14336, 16, 2, False)]
    return cases


@pytest.mark.parametrize("i,fmt,rows,cols,nx,pad,idx", make_cases())
def test_fastk_random_bitwise(flh, orc, gpu, i, fmt, rows, cols, nx, pad, idx):
    say("fastk", i, fmt, rows, cols, nx, pad, idx)
    rng = np.random.default_rng(500 + i)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    ys = rows + pad
    y0 = rng.standard_normal((nx - 1) * ys + rows).astype(np.float32)
    if idx:
        rb = rows * row_bytes(fmt, cols)
        ww = np.concatenate([sane_rows(fmt, rows, cols, rng), sane_rows(fmt, rows, cols, rng), w])
        got, want = run_dot(flh, orc, gpu, fmt, ww, rows, cols, xs, mode="f32fast", y0=y0, id_slot=2,
                            estride=rb, ystride=ys)
    else:
        got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode="f32fast", y0=y0, ystride=ys)
    assert np.array_equal(bits(got), bits(want))


def make_f32_cases(n=28, seed=91):
    """F32 and Q8_0 (one chain per lane over the whole row): columns of every
    kind (F32: below 16, not a multiple of 16 or 256; Q8_0: multiples of 32
    that end in a partial 256-column block; several activation tiles), 1-16
    columns, padding, the expert-slot form, router shapes (64 x 2048, 8 x 4096,
    160 x 5120)."""
    rng = np.random.default_rng(seed)
    colset = [1, 7, 15, 16, 17, 255, 256, 257, 1000, 2048, 4096, 5120, 8191, 9000, 20000]
    cases = []
    for i in range(2 * n):
        fmt = F32 if i < n else Q8_0
        cols = colset[rng.integers(len(colset))]
        if fmt == Q8_0:
            cols = max(32, cols // 32 * 32)
        rows = int(np.exp(rng.uniform(0, np.log(3000))))
        nx = 1 if rng.random() < 0.5 else int(rng.integers(2, 17))
        while rows * cols * max(1, nx // 4) > 6_000_000:
            rows = max(1, rows // 2)
        cases.append((i, fmt, rows, cols, nx, int(rng.integers(0, 3)), rng.random() < 0.2))
    cases += [(100, F32, 64, 2048, 1, 0, False), (101, F32, 8, 4096, 1, 0, True), (102, F32, 160, 5120, 1, 0, False),
              (103, F32, 64, 2048, 8, 1, False), (104, F32, 17, 40000, 1, 0, False), (105, F32, 33, 5000, 16, 2, False),
              (106, Q8_0, 4096, 4096, 1, 0, False), (107, Q8_0, 300, 14336, 3, 1, True), (108, Q8_0, 5, 32, 16, 0, False)]
    return cases


@pytest.mark.parametrize("i,fmt,rows,cols,nx,pad,idx", make_f32_cases())
def test_f32_q8_0_fast_random_bitwise(flh, orc, gpu, i, fmt, rows, cols, nx, pad, idx):
    say("f32/q8_0 fast", i, fmt, rows, cols, nx, pad, idx)
    rng = np.random.default_rng(900 + i)
    def weights():
        if fmt == F32:
            return normal_weights(rows, cols, rng, std=0.5).view(np.uint8).reshape(-1)
        return sane_rows(fmt, rows, cols, rng)
    w = weights()
    ys = rows + pad
    y0 = rng.standard_normal((nx - 1) * ys + rows).astype(np.float32)
    xs = activations(nx, cols, rng, outliers=True)
    st = col_stride_floats(cols)
    dx, hx = dev_cols(flh, gpu, xs, st)
    dy = flh.DeviceBuffer.from_array(y0, gpu)
    e, estride, ww = None, 0, w
    if idx:
        e, estride = 1, w.size
        ww = np.concatenate([weights(), w])
    dw = flh.DeviceBuffer.from_array(ww, gpu)
    slot = None if e is None else flh.DeviceBuffer.from_array(np.array([e], dtype=np.uint32), gpu)
    flh.stream_dot(fmt, dw, rows, cols, dx, dy, gpu, nx=nx, xstride=st, ystride=ys, id_slot=slot,
                   estride=estride, fast=True, i8_mask=0, i8k_mask=0)
    got = dy.download(np.float32, y0.size, gpu)
    want = y0.copy()
    orc.stream_dot(fmt, ww, rows, cols, hx, want, nx=nx, xstride=st, ystride=ys, fast=True, i8_mask=0,
                   i8k_mask=0, id_slot=e, estride=estride, threads=8)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", [F32, Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS])
@pytest.mark.parametrize("masks", [(0, 0), (I8, I8K), (I8 | 0b1100000, 0)])
def test_rows_of_no_columns(flh, orc, gpu, fmt, masks):
    """cols = 0 on every route (fp32, the default int8 masks, IQ on int8): every
    row's dot is 0 and y += 0 (-0 becomes +0), as the reference's loop over an
    empty row."""
    say("cols 0", fmt, masks)
    rows = 37
    y0 = np.array([-0.0, 1.5, -2.0] * 12 + [3.0], dtype=np.float32)
    dy = flh.DeviceBuffer.from_array(y0, gpu)
    dw = flh.DeviceBuffer.from_array(np.zeros(16, dtype=np.uint8), gpu)
    dx = flh.DeviceBuffer.from_array(np.zeros(64, dtype=np.float32), gpu)
    flh.stream_dot(fmt, dw, rows, 0, dx, dy, gpu, fast=True, i8_mask=masks[0], i8k_mask=masks[1], w_bytes=0)
    if fmt in (Q4_K, Q6_K) and masks == (I8, I8K):     # the fused ACT_Q8 entry point too
        flh.act_q8_stream_dot(fmt, dw, rows, 0, dx, dy, gpu)
    got = dy.download(np.float32, rows, gpu)
    assert np.array_equal(bits(got), bits(y0 + np.float32(0.0)))


def test_moe_rejects_rows_of_no_columns(flh, gpu):
    """The grouped expert entry points take cols as a positive multiple of 256:
    0 is an argument error, nothing launched."""
    d = flh.DeviceBuffer.from_array(np.zeros(64, dtype=np.float32), gpu)
    ids = flh.DeviceBuffer.from_array(np.zeros(4, dtype=np.uint32), gpu)
    with pytest.raises(flh.FlhError, match="positive multiple of 256"):
        flh.moe_dot(Q4_K, d, 256, 4, 0, ids, 1, 1, 2, d, 64, False, d, 4, gpu)
