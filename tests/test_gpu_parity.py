"""GPU parity: the HIP path against the C oracle (itself pinned to the
reference by tests/test_oracle_golden.py), through the C-ABI.

Bar: bitwise for ACT_Q8 bytes, dequant and every int8 / fp32 STREAM_DOT mode
(the kernels reproduce the reference's integer partials and float fold
order exactly).  Full BASELINE shapes are also checked bitwise; the
north-star tolerance (max |dy| <= 1e-3 * max |y| vs an f64 dequant dot) is
checked on top of that for the headline shapes.
"""
import os

import numpy as np
import pytest

from oracle import (Q8_0, Q4_K, Q6_K, col_stride_floats, row_bytes, x_alloc_bytes, xq_offset,
                    xqk_offset)
from util import tuned, sane_rows, normal_weights, activations

pytestmark = pytest.mark.gpu

I8 = 0b11110
I8K = 0b11000


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def say(*a):
    print("[case]", *a, flush=True)


def dev_cols(flh, gpu, xs, st):
    """Upload nx fp32 columns at stride st floats (appendix space zeroed)."""
    nx, cols = xs.shape
    buf = np.zeros(nx * st, dtype=np.float32)
    for p in range(nx):
        buf[p * st:p * st + cols] = xs[p]
    return flh.DeviceBuffer.from_array(buf, gpu), buf


def run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode="int8", y0=None, id_slot=None,
            estride=0, ystride=None):
    nx = xs.shape[0]
    st = col_stride_floats(cols)
    ys = rows if ystride is None else ystride
    fast, i8, i8k = {"int8": (1, I8, I8K), "q81": (1, I8, 0), "f32fast": (1, 0, 0),
                     "canon": (0, 0, 0), "iq8": (1, 0b1100000, 0)}[mode]
    dx, hx = dev_cols(flh, gpu, xs, st)
    flh.act_q8(dx, cols, gpu, nx=nx, xstride=st)
    xq = dx.download(np.float32, nx * st, gpu)
    ref_x = orc.act_q8_cols(xs, st)
    for p in range(nx):      # the device appendix equals the oracle's, byte for byte
        a = xq[p * st:(p * st) + x_alloc_bytes(cols) // 4].view(np.uint8)
        b = ref_x[p * st:(p * st) + x_alloc_bytes(cols) // 4].view(np.uint8)
        assert np.array_equal(a, b), f"act_q8 column {p}"
    yinit = np.zeros((nx - 1) * ys + rows, dtype=np.float32) if y0 is None else y0.copy()
    dy = flh.DeviceBuffer.from_array(yinit, gpu)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    slot = None
    if id_slot is not None:
        slot = flh.DeviceBuffer.from_array(np.array([id_slot], dtype=np.uint32), gpu)
    flh.stream_dot(fmt, dw, rows, cols, dx, dy, gpu, nx=nx, xstride=st, ystride=ys,
                   id_slot=slot, estride=estride, fast=fast, i8_mask=i8, i8k_mask=i8k)
    got = dy.download(np.float32, yinit.size, gpu)
    want = yinit.copy()
    orc.stream_dot(fmt, w, rows, cols, ref_x, want, nx=nx, xstride=st, ystride=ys, fast=fast,
                   i8_mask=i8, i8k_mask=i8k, id_slot=id_slot, estride=estride, threads=8)
    return got, want


# --------------------------------------------------------------- ACT_Q8 --
@pytest.mark.parametrize("cols", [32, 96, 256, 512, 2816, 4096, 14336])
def test_act_q8_bytes(flh, orc, gpu, cols):
    say("act_q8", cols)
    rng = np.random.default_rng(cols)
    xs = activations(3, cols, rng, outliers=True)
    xs[1, :64] = 0.0
    xs[2, 5:40] = 1e-41
    st = col_stride_floats(cols)
    dx, _ = dev_cols(flh, gpu, xs, st)
    flh.act_q8(dx, cols, gpu, nx=3, xstride=st)
    got = dx.download(np.float32, 3 * st, gpu)
    want = orc.act_q8_cols(xs, st)
    for p in range(3):
        n = x_alloc_bytes(cols)
        assert np.array_equal(got[p * st:].view(np.uint8)[:n], want[p * st:].view(np.uint8)[:n])


def test_act_q8_golden(flh, gpu, golden):
    for cols in (96, 256, 512, 2816, 4096):
        say("act_q8 golden", cols)
        x = golden[f"act_{cols}_x"]
        st = col_stride_floats(cols)
        dx, _ = dev_cols(flh, gpu, x[None, :], st)
        flh.act_q8(dx, cols, gpu)
        got = dx.download(np.uint8, x_alloc_bytes(cols), gpu)
        assert np.array_equal(got, golden[f"act_{cols}_buf"])


# --------------------------------------------------------------- dequant --
@pytest.mark.parametrize("fmt", [Q8_0, Q4_K, Q6_K])
@pytest.mark.parametrize("cols", [256, 2816, 4096])
def test_dequant_bitexact(flh, orc, gpu, fmt, cols):
    say("dequant", fmt, cols)
    rng = np.random.default_rng(fmt * 100 + cols)
    rows = 9
    w = sane_rows(fmt, rows, cols, rng)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    out = flh.DeviceBuffer(rows * cols * 4)
    flh.dequant(fmt, dw, rows, cols, out, gpu)
    got = out.download(np.float32, rows * cols, gpu)
    want = orc.dequant(fmt, w, rows, cols).ravel()
    assert np.array_equal(bits(got), bits(want))


def test_dequant_golden(flh, gpu, golden):
    for fmt, cols in [(Q8_0, 512), (Q4_K, 1024), (Q6_K, 1024)]:
        w = golden[f"dq_{fmt}_w"]
        dw = flh.DeviceBuffer.from_array(w, gpu)
        out = flh.DeviceBuffer(3 * cols * 4)
        flh.dequant(fmt, dw, 3, cols, out, gpu)
        got = out.download(np.float32, 3 * cols, gpu)
        assert np.array_equal(bits(got), bits(golden[f"dq_{fmt}_out"].ravel()))


def test_dequant_every_half_scale(flh, orc, gpu):
    """All 65536 fp16 scale patterns through the Q8_0 dequant (exact h2f)."""
    say("dequant all halves")
    nb = 65536
    w = np.zeros((nb, 34), dtype=np.uint8)
    w[:, 0:2] = np.arange(nb, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    w[:, 2:] = np.array([1, -1, 3, 127, -127, 0] + [2] * 26, dtype=np.int8).view(np.uint8)
    w = w.ravel()
    rows, cols = 2048, 1024
    dw = flh.DeviceBuffer.from_array(w, gpu)
    out = flh.DeviceBuffer(rows * cols * 4)
    flh.dequant(Q8_0, dw, rows, cols, out, gpu)
    got = out.download(np.float32, rows * cols, gpu)
    want = orc.dequant(Q8_0, w, rows, cols).ravel()
    g, h = bits(got), bits(want)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(g[~nan], h[~nan])


# ------------------------------------------------------- int8 STREAM_DOT --
SMALL_SHAPES = [(1, 256), (5, 512), (37, 1024), (64, 2048), (33, 2816), (17, 4096), (9, 14336)]


@pytest.mark.parametrize("fmt", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows,cols", SMALL_SHAPES)
def test_i8k_dot_bitwise_random_blocks(flh, orc, gpu, fmt, rows, cols):
    say("i8k random", fmt, rows, cols)
    rng = np.random.default_rng(rows * 7 + cols + fmt)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(1, cols, rng, outliers=True)
    y0 = rng.standard_normal(rows).astype(np.float32)
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, y0=y0)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("rows,cols", [(1, 32), (3, 96), (37, 1024), (64, 2048), (33, 2816),
                                       (17, 4096), (9, 14336), (5, 16384)])
def test_q8_0_dot_bitwise(flh, orc, gpu, rows, cols):
    say("q8_0", rows, cols)
    rng = np.random.default_rng(rows * 11 + cols)
    w = sane_rows(Q8_0, rows, cols, rng)
    xs = activations(1, cols, rng)
    y0 = rng.standard_normal(rows).astype(np.float32)
    got, want = run_dot(flh, orc, gpu, Q8_0, w, rows, cols, xs, y0=y0)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", [Q8_0, Q4_K, Q6_K])
@pytest.mark.parametrize("nx", [2, 3, 4, 5, 8, 16])
def test_multicol_bitwise_equals_single(flh, orc, gpu, fmt, nx):
    """nx-column tile == nx single tiles == oracle (fastllm.h:87-93)."""
    say("multicol", fmt, nx)
    rng = np.random.default_rng(nx * 3 + fmt)
    rows, cols = 45, 2048
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng)
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, ystride=rows + 3,
                        y0=np.zeros((nx - 1) * (rows + 3) + rows, dtype=np.float32))
    assert np.array_equal(bits(got), bits(want))
    for p in (0, nx - 1):
        g1, w1 = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs[p:p + 1])
        assert np.array_equal(bits(g1), bits(got[p * (rows + 3):p * (rows + 3) + rows]))


@pytest.mark.parametrize("fmt", [Q8_0, Q4_K, Q6_K])
@pytest.mark.parametrize("rows,nx", [(300, 2), (77, 3), (130, 4), (40, 8)])
def test_one_superblock_rows_multicol_bitwise(flh, orc, gpu, fmt, rows, nx):
    """Rows of a single 256-weight superblock with several columns: the
    streaming kernel's row / superblock split of a batch-local index
    (quotient by the superblocks per row, here 1) -- regression for a
    multiply-high divisor that does not fit 32 bits when it is 1."""
    say("one-superblock rows", fmt, rows, nx)
    cols = 256
    rng = np.random.default_rng(rows * 7 + nx + fmt)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, ystride=rows,
                        y0=rng.standard_normal((nx - 1) * rows + rows).astype(np.float32))
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", [Q4_K, Q6_K, Q8_0])
def test_idx_dot_resolves_expert_on_device(flh, orc, gpu, fmt):
    say("idx", fmt)
    rng = np.random.default_rng(99 + fmt)
    rows, cols, ne = 21, 1024, 4
    w = sane_rows(fmt, rows * ne, cols, rng)
    xs = activations(1, cols, rng)
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, id_slot=3,
                        estride=rows * row_bytes(fmt, cols))
    assert np.array_equal(bits(got), bits(want))


def test_i8k_golden_vectors(flh, gpu, golden):
    """The reference's own i8k / i8 outputs, through the device path."""
    n = int(golden["dot_count"][0])
    done = 0
    for i in range(n):
        fmt, cols, rows, nx, st, fast, i8, i8k = (int(v) for v in golden[f"dot{i}_meta"])
        say("golden dot", i, fmt, cols, nx, fast, i8, i8k)
        xb = golden[f"dot{i}_x"]
        dx = flh.DeviceBuffer.from_array(xb, gpu)
        dw = flh.DeviceBuffer.from_array(golden[f"dot{i}_w"], gpu)
        dy = flh.DeviceBuffer.from_array(golden[f"dot{i}_y0"], gpu)
        flh.stream_dot(fmt, dw, rows, cols, dx, dy, gpu, nx=nx, xstride=st, ystride=rows,
                       fast=fast, i8_mask=i8, i8k_mask=i8k)
        got = dy.download(np.float32, nx * rows, gpu)
        assert np.array_equal(bits(got), bits(golden[f"dot{i}_y"])), i
        done += 1
    assert done == n


@pytest.mark.parametrize("fmt", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows,cols,nx", [(7, 256, 1), (33, 2816, 1), (19, 4096, 3), (5, 14336, 2)])
def test_k_formats_on_q8_1_path_bitwise(flh, orc, gpu, fmt, rows, cols, nx):
    """Non-default masks (i8 bit without the i8k bit) route K formats to
    fl_dot_i8_q4_K / fl_dot_i8_q6_K (src/runtime/quants.h:468-526)."""
    say("q8_1 K path", fmt, rows, cols, nx)
    rng = np.random.default_rng(fmt * 31 + cols + nx)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode="q81")
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("mode", ["f32fast", "canon"])
@pytest.mark.parametrize("fmt", [Q8_0, Q4_K, Q6_K])
def test_fp32_modes_bitwise(flh, orc, gpu, mode, fmt):
    say("fp32 mode", mode, fmt)
    rng = np.random.default_rng(5 + fmt)
    rows, cols = 19, 1024
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(2, cols, rng)
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode=mode)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows,cols,nx", [(1, 256, 1), (5, 768, 16), (301, 2816, 3), (64, 16384, 2),
                                          (1027, 4096, 7), (3, 1280, 1)])
def test_fast_fp32_k_formats_wave_per_row(flh, orc, gpu, fmt, rows, cols, nx):
    """The fast fp32 order of the K formats on one wave per row (four chunks
    per pass, partial last pass, 1-16 columns, a row of one superblock and of
    64): bitwise against the oracle's dot_row_fast_dequant order, with old y."""
    say("fast fp32 k", fmt, rows, cols, nx)
    rng = np.random.default_rng(fmt + 3 * rows + cols + nx)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    y0 = rng.standard_normal((nx - 1) * (rows + 1) + rows).astype(np.float32)
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode="f32fast", y0=y0, ystride=rows + 1)
    assert np.array_equal(bits(got), bits(want))


# ----------------------------------------------------- BASELINE shapes --
@pytest.mark.parametrize("fmt,rows,cols", [
    (Q8_0, 4096, 4096),
    (Q4_K, 6144, 4096), (Q4_K, 4096, 4096), (Q4_K, 28672, 4096), (Q4_K, 4096, 14336),
    (Q6_K, 4096, 14336), (Q6_K, 128256, 4096)])
def test_baseline_shapes_bitwise_and_tolerance(flh, orc, gpu, fmt, rows, cols):
    """Device quantizer -> same bytes as host quantizer; matvec bitwise vs the
    oracle; error budget vs the f64 dequant dot."""
    say("baseline", fmt, rows, cols)
    rng = np.random.default_rng(rows + cols + fmt)
    n = rows * cols
    wf = flh.DeviceBuffer(n * 4)
    flh.fill_normal(wf, n, seed=1000 + fmt, stream=gpu, std=0.02)
    wq = flh.DeviceBuffer(rows * row_bytes(fmt, cols))
    flh.quantize(fmt, wf, rows, cols, wq, gpu)
    w = wq.download(np.uint8, rows * row_bytes(fmt, cols), gpu)
    if rows <= 8192:           # device quantizer == host quantizer, byte for byte
        wh = wf.download(np.float32, n, gpu).reshape(rows, cols)
        assert np.array_equal(flh.quantize_host(fmt, wh), w)
    wf.close()
    xs = activations(1, cols, rng, outliers=(fmt == Q4_K))
    got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs)
    assert np.array_equal(bits(got), bits(want))
    # north-star gate vs the reference int8 path (bitwise above implies 0 error)
    assert np.max(np.abs(got - want)) <= 1e-3 * np.max(np.abs(want))
    if rows <= 6144:
        # Mathematics pins the int8 path independently of the oracle's code:
        # it equals the f64 dot of the dequantised weights with the
        # dequantised activation (d_x * q per block of the appendix), up to
        # fp32 rounding of the fold.  Normalised per row by ||w .* x_hat||_2.
        deq = orc.dequant(fmt, w, rows, cols).astype(np.float64)
        xhat = dequant_activation(orc, xs[0], fmt)
        prod = deq * xhat[None, :]
        ref = prod.sum(axis=1)
        S = np.sqrt((prod ** 2).sum(axis=1))
        assert np.max(np.abs(got - ref) / np.maximum(S, 1e-6)) < 1e-4


def dequant_activation(orc, x, fmt):
    """x_hat from the ACT_Q8 appendix the kernel consumed: q8_K (d per 256)
    for K formats, q8_1 (f16 d per 32) for Q8_0."""
    cols = x.size
    buf = orc.act_q8(x)
    if fmt == Q8_0:
        blk = buf[xq_offset(cols):xq_offset(cols) + (cols // 32) * 36].reshape(-1, 36)
        d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)
        q = blk[:, 4:].view(np.int8).astype(np.float64)
        return (d * q).ravel()
    blk = buf[xqk_offset(cols):xqk_offset(cols) + (cols // 256) * 292].reshape(-1, 292)
    d = blk[:, 0:4].copy().view(np.float32).astype(np.float64)
    q = blk[:, 36:].view(np.int8).astype(np.float64)
    return (d * q).ravel()


# ------------------------------------------------ fused ACT_Q8 + STREAM_DOT --
@pytest.mark.parametrize("fmt", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows,cols,nx", [(37, 1024, 1), (300, 4096, 1), (64, 14336, 1), (300, 256, 2), (77, 256, 4),
                                          (33, 2816, 3), (20, 4096, 4), (1, 256, 2)])
def test_fused_act_q8_dot_bitwise(flh, orc, gpu, fmt, rows, cols, nx):
    """flh_act_q8_stream_dot == ACT_Q8 then STREAM_DOT: same appendix bytes
    in memory, bitwise-equal outputs (vs the oracle)."""
    say("fused act+dot", fmt, rows, cols, nx)
    rng = np.random.default_rng(rows + cols + nx + fmt)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    st = col_stride_floats(cols)
    dx, _ = dev_cols(flh, gpu, xs, st)
    y0 = rng.standard_normal((nx - 1) * rows + rows).astype(np.float32)
    dy = flh.DeviceBuffer.from_array(y0, gpu)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    flh.act_q8_stream_dot(fmt, dw, rows, cols, dx, dy, gpu, nx=nx, xstride=st, ystride=rows)
    got = dy.download(np.float32, y0.size, gpu)
    xq = dx.download(np.float32, nx * st, gpu)
    ref_x = orc.act_q8_cols(xs, st)
    for p in range(nx):
        n = x_alloc_bytes(cols) // 4
        assert np.array_equal(xq[p * st:p * st + n].view(np.uint8), ref_x[p * st:p * st + n].view(np.uint8))
    want = y0.copy()
    orc.stream_dot(fmt, w, rows, cols, ref_x, want, nx=nx, xstride=st, ystride=rows, threads=8)
    assert np.array_equal(bits(got), bits(want))


# ------------------------------------------- 8- and 4-wave streaming kernels --
@pytest.mark.parametrize("w8", ["15,2", "15,1", "0,2"])
@pytest.mark.parametrize("fmt,rows,cols", [(Q4_K, 1000, 4096), (Q6_K, 513, 14336), (Q4_K, 3, 2816),
                                           (Q8_0, 700, 4096), (Q6_K, 300, 512)])
def test_streaming_workgroup_shapes_bitwise(flh, orc, gpu, w8, fmt, rows, cols):
    """Every workgroup shape of the single-column streaming kernel (4 or 8
    waves, one or two per CU; FLH_KS_W8 = "mode bits,workgroups per CU"),
    fused with ACT_Q8 or not, equals the oracle bit for bit (Q4_K with the
    superblock-per-lane kernel switched off, so that this kernel runs)."""
    say("kstream shapes", w8, fmt, rows, cols)
    rng = np.random.default_rng(rows + cols + fmt)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(1, cols, rng, outliers=True)
    with tuned(flh, FLH_KS_W8=w8, FLH_SBL="0"):
        got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, y0=rng.standard_normal(rows).astype(np.float32))
        assert np.array_equal(bits(got), bits(want))
        if fmt != Q8_0:
            st = col_stride_floats(cols)
            dx, _ = dev_cols(flh, gpu, xs, st)
            dy = flh.DeviceBuffer.from_array(np.zeros(rows, np.float32), gpu)
            dw = flh.DeviceBuffer.from_array(w, gpu)
            flh.act_q8_stream_dot(fmt, dw, rows, cols, dx, dy, gpu)
            want2 = np.zeros(rows, np.float32)
            orc.stream_dot(fmt, w, rows, cols, orc.act_q8_cols(xs, st), want2, threads=8)
            assert np.array_equal(bits(dy.download(np.float32, rows, gpu)), bits(want2))
