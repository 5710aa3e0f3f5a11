"""Pins the C oracle with checks that do not use the reference's code.

The golden vectors (test_oracle_golden.py) pin the oracle to the reference's
own outputs; these tests pin it to what the mathematics and the format
definitions fix, each written independently of fl_oracle.c (numpy,
vectorised, exact rational arithmetic), chosen so that a dropped term, a
wrong shift / index or a swapped operand fails:
  * half2float: all 65536 halves vs numpy float16;
  * float2half: the reference KATs (tests/test_runtime.cpp:540-544) and
    numpy's round-to-nearest-even on random floats;
  * dequant: per-element transcription of the block layouts;
  * ACT_Q8: bsums = per-16 sums, d = amax/127, round-half-away quantisation;
  * int8 dots: integer partials from numpy int64, the reference fold order
    replayed with exactly-rounded fmaf (Fractions);
  * error budgets vs an f64 dot (tests/test_runtime.cpp:547-587, 687-723).
"""
from fractions import Fraction

import numpy as np
import pytest

from oracle import Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS, row_bytes, xq_offset, xqk_offset
from util import sane_rows


# ------------------------------------------------------------- fp16 --
def test_half2float_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([orc.half2float(int(v)) for v in h], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_float2half_kats_and_rne(orc):
    assert orc.float2half(1.0) == 0x3C00
    assert orc.float2half(-2.0) == 0xC000
    assert orc.float2half(65504.0) == 0x7BFF
    assert orc.float2half(1e30) == 0x7C00
    assert orc.float2half(5.96046448e-8) == 0x0001
    rng = np.random.default_rng(1)
    f = np.concatenate([(rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000)).astype(np.float32),
                        rng.integers(0, 1 << 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    f = f[~np.isnan(f)]
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    got = np.array([orc.float2half(float(v)) for v in f], dtype=np.uint16)
    assert np.array_equal(got, want)


# ----------------------------------------------------------- dequant --
def h16(b):
    return b.copy().view(np.float16).astype(np.float32)


def deq_reference_numpy(fmt, w, rows, cols):
    """Vectorised per-element decode of the block layouts (quants.h:23-26)."""
    if fmt == Q8_0:
        B = w.reshape(rows * cols // 32, 34)
        d = h16(B[:, 0:2])[:, 0]
        q = B[:, 2:].view(np.int8).astype(np.float32)
        return (d[:, None] * q).reshape(rows, cols)
    if fmt == Q5_0:
        B = w.reshape(rows * cols // 32, 22)
        d = h16(B[:, 0:2])[:, 0]
        qh = B[:, 2:6].copy().view("<u4")[:, 0].astype(np.uint64)
        qs = B[:, 6:22].astype(np.uint64)
        j = np.arange(16, dtype=np.uint64)
        lo = (qs & 0xF) | (((qh[:, None] >> j) & 1) << 4)           # element j: bit j of qh
        hi = (qs >> 4) | (((qh[:, None] >> (j + 16)) & 1) << 4)     # element 16 + j: bit 16 + j
        q = np.concatenate([lo, hi], axis=1).astype(np.float32) - 16.0
        return (d[:, None] * q).reshape(rows, cols)
    if fmt == Q4_K:
        B = w.reshape(rows * cols // 256, 144)
        d, dmin = h16(B[:, 0:2])[:, 0], h16(B[:, 2:4])[:, 0]
        s = B[:, 4:16].astype(np.uint32)
        sc = np.empty((len(B), 8), np.uint32)
        mn = np.empty((len(B), 8), np.uint32)
        sc[:, :4], mn[:, :4] = s[:, 0:4] & 63, s[:, 4:8] & 63
        sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
        mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
        qs = B[:, 16:].reshape(-1, 4, 32)
        nib = np.empty((len(B), 8, 32), np.float32)
        nib[:, 0::2] = (qs & 0xF).astype(np.float32)
        nib[:, 1::2] = (qs >> 4).astype(np.float32)
        d1 = d[:, None] * sc.astype(np.float32)
        m1 = dmin[:, None] * mn.astype(np.float32)
        return (d1[:, :, None] * nib - m1[:, :, None]).reshape(rows, cols)
    B = w.reshape(rows * cols // 256, 210)
    d = h16(B[:, 208:210])[:, 0]
    out = np.empty((len(B), 256), np.float32)
    for h in range(2):
        ql = B[:, 64 * h:64 * h + 64].astype(np.int32)
        qh = B[:, 128 + 32 * h:128 + 32 * h + 32].astype(np.int32)
        sc = B[:, 192 + 8 * h:200 + 8 * h].view(np.int8).astype(np.float32)
        for g in range(4):
            lb = ql[:, 32 * (g & 1):32 * (g & 1) + 32]
            lo = (lb & 0xF) if g < 2 else (lb >> 4)
            q6 = lo | (((qh >> (2 * g)) & 3) << 4)
            s16 = np.repeat(sc[:, 2 * g:2 * g + 2], 16, axis=1)
            out[:, 128 * h + 32 * g:128 * h + 32 * g + 32] = (d[:, None] * s16) * (q6 - 32).astype(np.float32)
    return out.reshape(rows, cols)


@pytest.mark.parametrize("fmt", [Q8_0, Q5_0, Q4_K, Q6_K])
def test_dequant_matches_format_definition(orc, fmt):
    rng = np.random.default_rng(fmt)
    rows, cols = 7, 1024
    w = sane_rows(fmt, rows, cols, rng)
    got = orc.dequant(fmt, w, rows, cols)
    want = deq_reference_numpy(fmt, w, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q4k_scale_unpack_every_byte(orc):
    """Each of the 8 (scale, min) pairs as a function of the 12 bytes: set one
    byte at a time to every value and compare with the closed form."""
    import ctypes as C
    for pos in range(12):
        for v in range(256):
            s = np.zeros(12, np.uint8)
            s[pos] = v
            for j in range(8):
                d, m = C.c_uint8(), C.c_uint8()
                orc.q4k_scale_min(j, s.ctypes.data, C.byref(d), C.byref(m))
                if j < 4:
                    ed, em = s[j] & 63, s[j + 4] & 63
                else:
                    ed = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4)
                    em = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
                assert (d.value, m.value) == (ed, em)


# ------------------------------------------------------------ ACT_Q8 --
def round_half_away(v):
    v = np.asarray(v, dtype=np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def test_act_q8_invariants(orc):
    rng = np.random.default_rng(5)
    cols = 1024
    x = rng.standard_normal(cols).astype(np.float32)
    x[rng.random(cols) < 0.02] *= 30
    x[256:512] = 0.0                                # an all-zero superblock
    buf = orc.act_q8(x)
    k = buf[xqk_offset(cols):xqk_offset(cols) + (cols // 256) * 292].reshape(-1, 292)
    for sb in range(cols // 256):
        xs = x[256 * sb:256 * sb + 256]
        amax = np.float32(np.max(np.abs(xs)))
        d = k[sb, 0:4].copy().view(np.float32)[0]
        assert d == np.float32(amax / np.float32(127))
        idv = np.float32(127) / amax if amax > 0 else np.float32(0)
        q = np.clip(round_half_away((xs * idv).astype(np.float32)), -127, 127).astype(np.int8)
        assert np.array_equal(k[sb, 36:].view(np.int8), q)
        bs = k[sb, 4:36].copy().view(np.int16)
        assert np.array_equal(bs, q.astype(np.int32).reshape(16, 16).sum(axis=1))
    blk = buf[xq_offset(cols):xq_offset(cols) + (cols // 32) * 36].reshape(-1, 36)
    for b in range(cols // 32):
        xs = x[32 * b:32 * b + 32]
        amax = np.float32(np.max(np.abs(xs)))
        d = np.float32(amax / np.float32(127))
        assert blk[b, 0:2].copy().view(np.float16)[0] == np.float16(d)
        q = blk[b, 4:].view(np.int8).astype(np.float32)
        assert np.all(np.abs(d * q - xs) <= amax / 127 + 1e-4 * max(amax, 1))


# ------------------------------------------------ exact fmaf fold replay --
def f32_round(fr: Fraction) -> np.float32:
    """Round an exact rational to the nearest float32, ties to even."""
    if fr == 0:
        return np.float32(0.0)
    c = np.float32(float(fr))                       # within one ulp of the answer
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        if not np.isfinite(cand):
            continue
        err = abs(Fraction(float(cand)) - fr)
        key = (err, int(np.float32(cand).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return np.float32(best[1])


def fmaf(a, b, c):
    return f32_round(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def fold4(a):
    s01 = np.float32(a[0] + a[1])
    s23 = np.float32(a[2] + a[3])
    return np.float32(s01 + s23)


def i8k_q4k_replay(row, xk, cols):
    """fl_dot_i8k_q4_K's contract (quants.h:528-561) restated from scratch."""
    nsb = cols // 256
    B = row.reshape(nsb, 144)
    X = xk.reshape(nsb, 292)
    s = B[:, 4:16].astype(np.int64)
    sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)], axis=1)
    mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
    qs = B[:, 16:].reshape(nsb, 4, 32).astype(np.int64)
    nib = np.empty((nsb, 8, 32), np.int64)
    nib[:, 0::2], nib[:, 1::2] = qs & 0xF, qs >> 4
    xq = X[:, 36:].view(np.int8).astype(np.int64).reshape(nsb, 8, 32)
    bs = X[:, 4:36].copy().view(np.int16).astype(np.int64).reshape(nsb, 8, 2).sum(axis=2)
    iacc = (sc * (nib * xq).sum(axis=2)).sum(axis=1)
    imin = (mn * bs).sum(axis=1)
    d, dmin = h16(B[:, 0:2])[:, 0], h16(B[:, 2:4])[:, 0]
    dk = X[:, 0:4].copy().view(np.float32)[:, 0]
    a = [np.float32(0)] * 4
    for sb in range(nsb):
        a[sb & 3] = fmaf(np.float32(d[sb] * dk[sb]), np.float32(iacc[sb]), a[sb & 3])
        a[sb & 3] = fmaf(-np.float32(dmin[sb] * dk[sb]), np.float32(imin[sb]), a[sb & 3])
    return fold4(a)


def i8k_q6k_replay(row, xk, cols):
    """fl_dot_i8k_q6_K's contract (quants.h:563-594) restated from scratch."""
    nsb = cols // 256
    B = row.reshape(nsb, 210)
    X = xk.reshape(nsb, 292)
    q6 = np.empty((nsb, 256), np.int64)
    for h in range(2):
        ql = B[:, 64 * h:64 * h + 64].astype(np.int64)
        qh = B[:, 128 + 32 * h:160 + 32 * h].astype(np.int64)
        for g in range(4):
            lb = ql[:, 32 * (g & 1):32 * (g & 1) + 32]
            q6[:, 128 * h + 32 * g:128 * h + 32 * g + 32] = ((lb & 0xF) if g < 2 else (lb >> 4)) | (((qh >> (2 * g)) & 3) << 4)
    xq = X[:, 36:].view(np.int8).astype(np.int64)
    idot = (q6 * xq).reshape(nsb, 16, 16).sum(axis=2)
    bs = X[:, 4:36].copy().view(np.int16).astype(np.int64)
    sc = B[:, 192:208].view(np.int8).astype(np.int64)
    iacc = (sc * (idot - 32 * bs)).sum(axis=1)
    d = h16(B[:, 208:210])[:, 0]
    dk = X[:, 0:4].copy().view(np.float32)[:, 0]
    a = [np.float32(0)] * 4
    for sb in range(nsb):
        a[sb & 3] = fmaf(np.float32(d[sb] * dk[sb]), np.float32(iacc[sb]), a[sb & 3])
    return fold4(a)


def i8_q80_replay(row, xq, cols):
    """fl_dot_i8_q8_0's contract (quants.h:438-447) restated from scratch."""
    nb = cols // 32
    B = row.reshape(nb, 34)
    X = xq.reshape(nb, 36)
    idot = (B[:, 2:].view(np.int8).astype(np.int64) * X[:, 4:].view(np.int8).astype(np.int64)).sum(axis=1)
    dd = h16(B[:, 0:2])[:, 0] * h16(X[:, 0:2])[:, 0]
    a = [np.float32(0)] * 4
    for b in range(nb):
        a[b & 3] = fmaf(np.float32(dd[b]), np.float32(idot[b]), a[b & 3])
    return fold4(a)


def i8_q50_replay(row, xq, cols):
    """fl_dot_i8_q5_0's contract (quants.h:449-466) restated from scratch:
    per block, the exact integer sum of (5-bit value - 16) * x, scaled by
    d_w * d_x (exact product of two halves), chained with fmaf into a4[b & 3]."""
    nb = cols // 32
    B = row.reshape(nb, 22)
    X = xq.reshape(nb, 36)
    d = h16(B[:, 0:2])[:, 0]
    q = deq_reference_numpy(Q5_0, row, 1, cols).reshape(nb, 32) / d[:, None]   # exact: q * d / d
    t = (np.rint(q).astype(np.int64) * X[:, 4:].view(np.int8).astype(np.int64)).sum(axis=1)
    dd = d * h16(X[:, 0:2])[:, 0]
    a = [np.float32(0)] * 4
    for b in range(nb):
        a[b & 3] = fmaf(np.float32(dd[b]), np.float32(t[b]), a[b & 3])
    return fold4(a)


@pytest.mark.parametrize("fmt,cols", [(Q4_K, 512), (Q4_K, 2816), (Q6_K, 1024), (Q6_K, 2304),
                                      (Q8_0, 512), (Q8_0, 1056), (Q5_0, 512), (Q5_0, 1408)])
def test_int8_dot_replay_bitwise(orc, fmt, cols):
    rng = np.random.default_rng(fmt * 7 + cols)
    rows = 5
    w = sane_rows(fmt, rows, cols, rng)
    x = rng.uniform(-1, 1, cols).astype(np.float32)
    x[rng.random(cols) < 0.01] *= 20
    buf = orc.act_q8(x)
    xk = buf[xqk_offset(cols):xqk_offset(cols) + (cols // 256) * 292]
    xq = buf[xq_offset(cols):xq_offset(cols) + (cols // 32) * 36]
    rb = row_bytes(fmt, cols)
    for r in range(rows):
        row = w[r * rb:(r + 1) * rb]
        if fmt == Q4_K:
            got, want = orc.dot_i8k_q4_K(row.ctypes.data, xk.ctypes.data, cols), i8k_q4k_replay(row, xk, cols)
        elif fmt == Q6_K:
            got, want = orc.dot_i8k_q6_K(row.ctypes.data, xk.ctypes.data, cols), i8k_q6k_replay(row, xk, cols)
        elif fmt == Q5_0:
            got, want = orc.dot_i8_q5_0(row.ctypes.data, xq.ctypes.data, cols), i8_q50_replay(row, xq, cols)
        else:
            got, want = orc.dot_i8_q8_0(row.ctypes.data, xq.ctypes.data, cols), i8_q80_replay(row, xq, cols)
        assert np.float32(got).view(np.uint32) == np.float32(want).view(np.uint32), (r, got, want)


# ------------------------------------------------------- error budgets --
@pytest.mark.parametrize("fmt,i8k,max_gate", [(Q4_K, True, 3e-2), (Q6_K, True, 3e-2),
                                             (Q8_0, False, 2.5e-2), (Q4_K, False, 2.5e-2),
                                             (Q6_K, False, 2.5e-2)])
def test_int8_error_budget_vs_f64(orc, fmt, i8k, max_gate):
    """The reference's own budgets: x ~ U(-1,1), cols 512, 200 trials, error
    normalised by ||w .* x||_2 (tests/test_runtime.cpp:547-587, 687-723)."""
    rng = np.random.default_rng(100 + fmt + 10 * i8k)
    cols, trials = 512, 200
    mx = mean = mcn = 0.0
    for _ in range(trials):
        w = sane_rows(fmt, 1, cols, rng)
        x = rng.uniform(-1, 1, cols).astype(np.float32)
        xb = orc.act_q8_cols(x[None, :])
        deq = orc.dequant(fmt, w, 1, cols)[0].astype(np.float64)
        prod = deq * x.astype(np.float64)
        ref, S = prod.sum(), max(1e-6, np.sqrt((prod ** 2).sum()))
        y = np.zeros(1, np.float32)
        orc.stream_dot(fmt, w, 1, cols, xb, y, i8_mask=0b11110, i8k_mask=0b11000 if i8k else 0)
        yc = np.zeros(1, np.float32)
        orc.stream_dot(fmt, w, 1, cols, xb, yc, fast=False)
        e = abs(float(y[0]) - ref) / S
        mx, mean = max(mx, e), mean + e / trials
        mcn = max(mcn, abs(float(yc[0]) - ref) / S)
    assert mx < max_gate and mean < 6e-3 and mcn < 1e-5, (mx, mean, mcn)


def test_multicolumn_equals_single_columns(orc):
    """fastllm.h:87-93: an nx-column tile equals nx single tiles, bitwise."""
    rng = np.random.default_rng(11)
    for fmt, cols in ((Q4_K, 1024), (Q6_K, 1024), (Q8_0, 1024)):
        rows, nx = 9, 5
        w = sane_rows(fmt, rows, cols, rng)
        xs = rng.uniform(-1, 1, (nx, cols)).astype(np.float32)
        xb = orc.act_q8_cols(xs)
        st = xb.size // nx
        y = np.zeros(nx * rows, np.float32)
        orc.stream_dot(fmt, w, rows, cols, xb, y, nx=nx, xstride=st, ystride=rows)
        for p in range(nx):
            y1 = np.zeros(rows, np.float32)
            orc.stream_dot(fmt, w, rows, cols, xb[p * st:(p + 1) * st], y1)
            assert np.array_equal(y[p * rows:(p + 1) * rows].view(np.uint32), y1.view(np.uint32))


def test_router_ties_and_norm(orc):
    ids, g = orc.router_sel(np.array([1.0, 3.0, 3.0, 0.5, 3.0], np.float32), 3, norm=1)
    assert list(ids) == [1, 2, 4]
    assert abs(float(g.sum()) - 1.0) < 1e-6
    ids, g = orc.router_sel(np.array([0.0, 0.0, 0.0, 0.0], np.float32), 2, norm=0, scale=2.0)
    assert list(ids) == [0, 1] and np.allclose(g, [0.5, 0.5])


# ----------------------------------------------------- IQ codebook formats --
def iq_grids():
    """The codebook values as written in the product header (their digest
    is pinned to the reference's tables in test_oracle_golden.py)."""
    import os
    import re
    src = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                            "fast-llm_amd", "csrc", "flh_iq_grids.h")).read()
    g2 = src.split("FLH_IQ2XXS_GRID_VALUES")[1].split("#define")[0]
    g3 = src.split("FLH_IQ3XXS_GRID_VALUES")[1]
    g2 = np.array([int(v, 16) for v in re.findall(r"0x([0-9a-f]+)ull", g2)], dtype=np.uint64)
    g3 = np.array([int(v, 16) for v in re.findall(r"0x([0-9a-f]+)u", g3)], dtype=np.uint32)
    assert g2.size == 256 and g3.size == 256
    return g2, g3


def iq_decode_numpy(fmt, row, cols):
    """Per 32-element group: db (float32, as (d * (0.5 + s)) * 0.25 or 0.5)
    and the 32 signed grid magnitudes (quants.h:237-290), vectorised."""
    g2, g3 = iq_grids()
    bb = 66 if fmt == IQ2_XXS else 98
    B = row.reshape(cols // 256, bb)
    d = h16(B[:, 0:2])[:, 0]
    if fmt == IQ2_XXS:
        W = B[:, 2:].reshape(-1, 8, 8)                       # [sb, group, 8 bytes]
        idx = W[:, :, 0:4].astype(np.int64)                  # grid index of run l
        w1 = W[:, :, 4:8].copy().view("<u4")[..., 0].astype(np.uint64)
        mag = ((g2[idx][..., None] >> (8 * np.arange(8, dtype=np.uint64))) & 0xFF).astype(np.int64)
        mag = mag.reshape(-1, 8, 32)                         # element 8l + j
        scale = 0.25
    else:
        qs = B[:, 2:66].reshape(-1, 8, 8).astype(np.int64)   # [sb, group, 8 indices]
        w1 = B[:, 66:98].copy().view("<u4").reshape(-1, 8).astype(np.uint64)
        ent = ((g3[qs][..., None] >> (8 * np.arange(4, dtype=np.uint32))) & 0xFF).astype(np.int64)
        mag = ent.reshape(-1, 8, 32)                         # entry 2l+h, byte j -> 8l + 4h + j
        scale = 0.5
    l = np.arange(32) // 8
    j = np.arange(32) % 8
    s7 = (w1[..., None] >> (7 * l).astype(np.uint64)) & 127
    par = np.zeros_like(s7)
    for b in range(7):
        par ^= (s7 >> b) & 1
    sgn = s7 | (par << 7)
    neg = (sgn >> j.astype(np.uint64)) & 1
    val = np.where(neg == 1, -mag, mag)
    sc = (w1 >> 28).astype(np.float32)
    db = (d[:, None] * (np.float32(0.5) + sc)) * np.float32(scale)
    return db.reshape(-1).astype(np.float32), val.reshape(-1, 32)


@pytest.mark.parametrize("fmt", [IQ2_XXS, IQ3_XXS])
def test_iq_dequant_and_canonical_order(orc, fmt):
    """dequant = db * (+-grid byte); the canonical dot is the single chain
    acc += (db * v) * x in the element order of quants.h:237-290 (IQ3: 8l+j
    then 8l+j+4), replayed in float32."""
    rng = np.random.default_rng(40 + fmt)
    rows, cols = 3, 512
    w = sane_rows(fmt, rows, cols, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    got = orc.dequant(fmt, w, rows, cols)
    rb = row_bytes(fmt, cols)
    order = [8 * l + j for l in range(4) for j in range(8)] if fmt == IQ2_XXS else \
        [8 * l + j + 4 * h for l in range(4) for j in range(4) for h in range(2)]
    for r in range(rows):
        db, val = iq_decode_numpy(fmt, w[r * rb:(r + 1) * rb], cols)
        want = (db[:, None] * val.astype(np.float32)).reshape(-1)
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32))
        acc = np.float32(0)
        for g in range(cols // 32):
            for e in order:
                acc = np.float32(acc + np.float32(np.float32(db[g] * np.float32(val[g, e])) * x[32 * g + e]))
        y = np.zeros(1, np.float32)
        orc.stream_dot(fmt, w[r * rb:(r + 1) * rb], 1, cols, x, y, fast=False)
        assert y[0].view(np.uint32) == acc.view(np.uint32)


@pytest.mark.parametrize("fmt", [IQ2_XXS, IQ3_XXS])
def test_iq_int8_replay_and_budget(orc, fmt):
    """q8_1 dot: exact integer group sums (numpy int64) folded with exactly
    rounded fmaf into a[b & 3]; and its error against an f64 dot stays in the
    budget the reference holds its q8_1 dots to (test_runtime.cpp:547-587)."""
    rng = np.random.default_rng(50 + fmt)
    cols = 1024
    mx = 0.0
    for t in range(60):
        w = sane_rows(fmt, 1, cols, rng)
        x = rng.uniform(-1, 1, cols).astype(np.float32)
        buf = orc.act_q8(x)
        xq = buf[xq_offset(cols):xq_offset(cols) + (cols // 32) * 36]
        X = xq.reshape(-1, 36)
        db, val = iq_decode_numpy(fmt, w, cols)
        idot = (val * X[:, 4:].view(np.int8).astype(np.int64)).sum(axis=1)
        dx = h16(X[:, 0:2])[:, 0]
        a = [np.float32(0)] * 4
        for b in range(cols // 32):
            a[b & 3] = fmaf(np.float32(db[b] * dx[b]), np.float32(idot[b]), a[b & 3])
        want = fold4(a)
        got = orc.dot_i8_iq(fmt, w.ctypes.data, xq.ctypes.data, cols)
        assert np.float32(got).view(np.uint32) == np.float32(want).view(np.uint32), t
        prod = (db[:, None].astype(np.float64) * val).reshape(-1) * x.astype(np.float64)
        S = max(1e-6, np.sqrt((prod ** 2).sum()))
        mx = max(mx, abs(float(got) - prod.sum()) / S)
    assert mx < 2.5e-2, mx


def test_device_round_half_away_identity():
    """The device quantizers round y = x * id with trunc(y + copysign(0.5 -
    2^-25, y)) (one add and a truncating convert) instead of roundf(y), then
    clamp to +-127 (fl_quantize_q8_1_block / fl_quantize_q8_K_block,
    src/runtime/quants.h:360-402).  Pinned here on every float within 2^13
    ulps of each integer and each half-integer in [-129, 129] -- where a
    wrong offset or a double rounding would show -- and on 2^20 random floats
    in that range, against roundf(y) = sign(y) * floor(|y| + 0.5) computed
    exactly in float64.  (Checked exhaustively over all floats with |y| <=
    128.5 when the identity was adopted.)"""
    c = np.float32(0.5) - np.float32(2.0 ** -25)
    assert c == np.float32(0.49999997)
    centers = np.concatenate([np.arange(0, 130, dtype=np.float32), np.arange(0, 129, dtype=np.float32) + 0.5])
    k = np.arange(-(1 << 13), 1 << 13, dtype=np.int64)
    ys = []
    for m in centers:
        b = np.int64(np.float32(m).view(np.int32)) + k
        b = b[(b >= 0) & (b < 0x43020000)]
        ys.append(b.astype(np.uint32).view(np.float32))
    ys.append(np.random.default_rng(3).uniform(0, 129, 1 << 20).astype(np.float32))
    y = np.concatenate(ys)
    y = np.concatenate([y, -y])
    with np.errstate(over="ignore"):
        t = (y + np.copysign(c, y)).astype(np.float32)
    got = np.clip(np.trunc(t).astype(np.int64), -127, 127)
    y64 = y.astype(np.float64)
    want = np.clip(np.sign(y64) * np.floor(np.abs(y64) + 0.5), -127, 127).astype(np.int64)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n", [256, 4096, 14336])
def test_rmsnorm_oracle_pinned(n):
    """orc_rmsnorm restates fl_op_rmsnorm (decode_params.h:101-106): the
    squares summed in order with one rounding each (numpy's float32 cumsum is
    that sequential sum), s = 1 / sqrt(mean + eps) correctly rounded, y =
    (x * s) * w -- bit for bit."""
    from oracle import Oracle
    o = Oracle()
    rng = np.random.default_rng(n + 1)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    ss = np.cumsum((x * x).astype(np.float32), dtype=np.float32)[-1]
    s = np.float32(1.0) / np.sqrt(np.float32(ss / np.float32(n) + np.float32(1e-5)), dtype=np.float32)
    want = ((x * s).astype(np.float32) * w).astype(np.float32)
    assert np.array_equal(o.rmsnorm(x, w, 1e-5).view(np.uint32), want.view(np.uint32))
