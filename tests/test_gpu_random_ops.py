"""Seeded random inputs for the non-matvec entry points.

ACT_Q8 (any multiple of 32 columns, 1-6 columns at padded strides, zero,
tiny and outlier blocks), dequant (every format), RMSNORM -> ACT_Q8 -> dot
in one call (every K and 32-weight-block format, random widths), SILU_MUL +
ACT_Q8, the router (2-128 experts, top-1..8, both normalisations, ties) and
WMERGE: bitwise against the oracle where the reference's arithmetic is
exact (appendix bytes, dequant values, ids, dots of the stored column,
WMERGE), within the documented tolerance where it calls expf (gates, silu)
or sums in order on the CPU (RMSNORM: the sequential-sum bound).
"""
import numpy as np
import pytest

from oracle import (Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS, col_stride_floats, row_bytes,
                    x_alloc_bytes)
from util import sane_rows, activations
from test_gpu_parity import bits, say, dev_cols

pytestmark = pytest.mark.gpu

FMTS = [Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS]
BLOCK = {Q8_0: 32, Q5_0: 32, Q4_K: 256, Q6_K: 256, IQ2_XXS: 256, IQ3_XXS: 256}


@pytest.mark.parametrize("seed", range(16))
def test_random_act_q8_bytes(flh, orc, gpu, seed):
    rng = np.random.default_rng(300 + seed)
    cols = 32 * int(rng.integers(1, 513))
    nx = int(rng.integers(1, 7))
    pad = 4 * int(rng.integers(0, 5))
    st = col_stride_floats(cols) + pad
    xs = activations(nx, cols, rng, outliers=True)
    for p in range(nx):                        # zero, subnormal and huge blocks
        if rng.random() < 0.5:
            b = int(rng.integers(0, cols // 32))
            xs[p, 32 * b:32 * b + 32] = [0.0, 1e-41, -3e38, 1e-30][int(rng.integers(0, 4))]
    say("random act_q8", seed, cols, nx, st)
    dx, _ = dev_cols(flh, gpu, xs, st)
    flh.act_q8(dx, cols, gpu, nx=nx, xstride=st)
    got = dx.download(np.float32, nx * st, gpu)
    want = orc.act_q8_cols(xs, st)
    for p in range(nx):
        a = got[p * st:p * st + x_alloc_bytes(cols) // 4].view(np.uint8)
        b = want[p * st:p * st + x_alloc_bytes(cols) // 4].view(np.uint8)
        assert np.array_equal(a, b), f"column {p}"


@pytest.mark.parametrize("seed", range(12))
def test_random_dequant_bitwise(flh, orc, gpu, seed):
    rng = np.random.default_rng(400 + seed)
    fmt = FMTS[seed % len(FMTS)]
    cols = BLOCK[fmt] * int(rng.integers(1, 64 if BLOCK[fmt] == 256 else 512))
    rows = int(rng.integers(1, 300))
    say("random dequant", seed, fmt, rows, cols)
    w = sane_rows(fmt, rows, cols, rng)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    out = flh.DeviceBuffer(rows * cols * 4)
    flh.dequant(fmt, dw, rows, cols, out, gpu)
    got = out.download(np.float32, rows * cols, gpu)
    assert np.array_equal(bits(got), bits(orc.dequant(fmt, w, rows, cols).ravel()))


@pytest.mark.parametrize("seed", range(16))
def test_random_rmsnorm_stream_dot(flh, orc, gpu, seed):
    """One call (one launch where a kernel takes the shape) equals
    rmsnorm_act_q8 + stream_dot bit for bit; the column is within the
    sequential-sum bound of the reference's; the dot equals the oracle's on
    the stored column."""
    rng = np.random.default_rng(500 + seed)
    fmt = [Q4_K, Q4_K, Q4_K, Q6_K, Q8_0, Q5_0][seed % 6]
    n = 256 * int(rng.integers(1, 57))
    rows = int(np.exp(rng.uniform(0, np.log(30000))))
    while rows * n > 60_000_000:
        rows //= 2
    say("random rmsnorm dot", seed, fmt, rows, n)
    x = (rng.standard_normal(n) * rng.uniform(0.1, 10)).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    w = sane_rows(fmt, rows, n, rng)
    y0 = rng.standard_normal(rows).astype(np.float32)
    st = col_stride_floats(n)
    dx, dwn, dw = (flh.DeviceBuffer.from_array(a, gpu) for a in (x, wn, w))
    outs = []
    for one in (True, False):
        dxn = flh.DeviceBuffer.from_array(np.zeros(st, np.float32), gpu)
        dy = flh.DeviceBuffer.from_array(y0, gpu)
        if one:
            flh.rmsnorm_stream_dot(fmt, dw, rows, n, dx, dwn, 1e-5, dxn, dy, gpu)
        else:
            flh.rmsnorm_act_q8(dx, dwn, dxn, n, 1e-5, gpu)
            flh.stream_dot(fmt, dw, rows, n, dxn, dy, gpu)
        outs.append((dxn.download(np.float32, st, gpu), dy.download(np.float32, rows, gpu)))
    (xa, ya), (xb, yb) = outs
    assert np.array_equal(bits(xa), bits(xb))
    assert np.array_equal(bits(ya), bits(yb))
    ref = orc.rmsnorm(x, wn, 1e-5)
    ulp = np.spacing(np.abs(ref))
    assert np.all(np.abs(xa[:n] - ref) <= n * 2.0 ** -24 * np.abs(ref) + 2 * ulp)
    want = y0.copy()
    orc.stream_dot(fmt, w, rows, n, xa, want, threads=8)
    assert np.array_equal(bits(ya), bits(want))


@pytest.mark.parametrize("seed", range(8))
def test_random_silu_mul_act_q8(flh, orc, gpu, seed):
    """SILU_MUL + ACT_Q8 in one launch: h within the expf tolerance of the
    reference's silu (fl_op_silu_mul, decode_params.h:267-272) and the
    appendices equal ACT_Q8 of the stored h byte for byte."""
    rng = np.random.default_rng(600 + seed)
    n = 256 * int(rng.integers(1, 57))
    ncol = int(rng.integers(1, 5))
    gs = 2 * n + 4 * int(rng.integers(0, 5))
    st = col_stride_floats(n)
    say("random silu", seed, n, ncol)
    gu = (rng.standard_normal(ncol * gs) * 4).astype(np.float32)
    dgu = flh.DeviceBuffer.from_array(gu, gpu)
    dh = flh.DeviceBuffer.from_array(np.zeros(ncol * st, np.float32), gpu)
    flh.silu_mul_act_q8(dgu, dgu.ptr + 4 * n, dh, n, ncol, gs, st, gpu)
    h = dh.download(np.float32, ncol * st, gpu)
    for c in range(ncol):
        g, u = gu[c * gs:c * gs + n], gu[c * gs + n:c * gs + 2 * n]
        hc = h[c * st:c * st + n]
        assert np.allclose(hc, orc.silu_mul(g, u), rtol=4e-7, atol=1e-30)
        app = orc.act_q8(hc).view(np.uint8)
        assert np.array_equal(h[c * st:c * st + x_alloc_bytes(n) // 4].view(np.uint8), app)


@pytest.mark.parametrize("seed", range(12))
def test_random_router(flh, orc, gpu, seed):
    rng = np.random.default_rng(700 + seed)
    E = int(rng.integers(2, 129))
    K = int(rng.integers(1, min(E, 8) + 1))
    ntok = int(rng.integers(1, 33))
    norm = int(rng.integers(0, 2))
    say("random router", seed, E, K, ntok, norm)
    logits = rng.standard_normal((ntok, E)).astype(np.float32)
    if rng.random() < 0.5:                     # ties: lower id first
        logits[:, 1::3] = logits[:, 0:1]
    dl = flh.DeviceBuffer.from_array(logits, gpu)
    di, dg = flh.DeviceBuffer(4 * ntok * K), flh.DeviceBuffer(4 * ntok * K)
    flh.router_sel(dl, ntok, E, K, norm, 1.0, di, dg, gpu)
    ids = di.download(np.uint32, ntok * K, gpu).reshape(ntok, K)
    gates = dg.download(np.float32, ntok * K, gpu).reshape(ntok, K)
    for t in range(ntok):
        wi, wg = orc.router_sel(logits[t], K, norm=norm)
        assert np.array_equal(ids[t], wi)
        assert np.allclose(gates[t], wg, rtol=2e-6, atol=1e-30)


@pytest.mark.parametrize("seed", range(8))
def test_random_wmerge(flh, orc, gpu, seed):
    rng = np.random.default_rng(800 + seed)
    n_parts = int(rng.integers(1, 9))
    n = int(rng.integers(1, 20000))
    # n_full: the full expert count of a truncated merge (the gates array
    # holds n_full entries, the first n_parts of them merged)
    n_full = n_parts + int(rng.integers(1, 5)) if rng.random() < 0.4 else 0
    scale = float(rng.uniform(0.5, 2.0))
    with_add = bool(rng.random() < 0.5)
    say("random wmerge", seed, n_parts, n, n_full, with_add)
    parts = rng.standard_normal((n_parts, n)).astype(np.float32)
    gates = rng.random(max(n_parts, n_full)).astype(np.float32)
    add1 = rng.standard_normal(n).astype(np.float32) if with_add else None
    dp = flh.DeviceBuffer.from_array(parts, gpu)
    dgt = flh.DeviceBuffer.from_array(gates, gpu)
    da = flh.DeviceBuffer.from_array(add1, gpu) if with_add else None
    dy = flh.DeviceBuffer(4 * n)
    flh.wmerge(dp, dgt, da, None, dy, scale, n_parts, n, n_full, 1, 0, 0, gpu)
    want = orc.wmerge(parts, gates, add1, None, scale=scale, n_full=n_full)
    assert np.array_equal(bits(dy.download(np.float32, n, gpu)), bits(want))
