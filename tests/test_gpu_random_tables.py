"""Seeded random task tables through flh_exec_tasks, bitwise against the oracle.

Each table holds, for one activation width, the ACT_Q8 of every activation
column and the STREAM_DOT / STREAM_DOT_IDX row tiles of a few matrices in
random formats (Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS), tile sizes,
column counts (1-4 columns of a group at the column stride) and orders,
the way the reference's graph builder cuts them (src/model/decoder.cpp:
482-528): an ACT_Q8 followed directly by a one-column q8_K tile of its
activation, consecutive tiles of one matrix and tiles of 2-byte aligned
rows all reach the adapter's fused and merged launches.  Every tile's
output must equal the oracle's exec_task_cpu result for that tile
(src/runtime/kernels.h:1002-1258), bit for bit.
"""
import numpy as np
import pytest

from oracle import Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS, col_stride_floats, row_bytes
from util import sane_rows, activations
from test_gpu_tasks import mk, bits

pytestmark = pytest.mark.gpu

FMTS = [Q4_K, Q4_K, Q6_K, Q6_K, Q8_0, Q5_0, IQ2_XXS, IQ3_XXS]
I8_ALL = 0b1111110          # every int8 format on its q8_1 / q8_K route


def make_table(seed):
    rng = np.random.default_rng(seed)
    cols = int(rng.choice([256, 512, 1024, 2304, 2816, 4096, 5120]))
    ncol = int(rng.integers(1, 5))               # activation columns
    mats = []
    for m in range(int(rng.integers(2, 6))):
        fmt = int(FMTS[rng.integers(len(FMTS))])
        rows = int(rng.integers(1, 2500))
        nx = int(rng.integers(1, ncol + 1))
        p0 = int(rng.integers(0, ncol - nx + 1))   # first activation column
        idx = rng.random() < 0.2
        ntile = int(rng.integers(1, 5))
        cuts = sorted(set(int(c) for c in rng.integers(1, rows, size=ntile - 1))) if rows > 1 else []
        bounds = [0] + cuts + [rows]
        mats.append(dict(fmt=fmt, rows=rows, nx=nx, p0=p0, idx=idx, tiles=list(zip(bounds[:-1], bounds[1:]))))
    # order: every ACT_Q8 first, except that one matrix's first tile may
    # directly follow the ACT_Q8 of its column (the adapter's fused pair)
    order = list(range(ncol))
    rng.shuffle(order)
    return cols, ncol, mats, order


CASES = list(range(48))


def build(flh, gpu, seed, y_zero=False):
    """The seeded table, its device buffers and host copies (old y zero with
    y_zero, so that a captured graph can reset it with a fill kernel)."""
    cols, ncol, mats, order = make_table(seed)
    rng = np.random.default_rng(10_000 + seed)
    st = col_stride_floats(cols)
    xs = activations(ncol, cols, rng, outliers=True)
    xb = np.zeros(ncol * st, np.float32)
    for p in range(ncol):
        xb[p * st:p * st + cols] = xs[p]
    dx = flh.DeviceBuffer.from_array(xb, gpu)
    T = flh.TaskKind
    tasks = []
    for m in mats:
        nmat = 3 if m["idx"] else 1
        w = sane_rows(m["fmt"], nmat * m["rows"], cols, rng)
        m["w"] = w
        m["dw"] = flh.DeviceBuffer.from_array(w, gpu)
        m["slot"] = flh.DeviceBuffer.from_array(np.array([2], np.uint32), gpu) if m["idx"] else None
        ny = (m["nx"] - 1) * m["rows"] + m["rows"]
        m["y0"] = np.zeros(ny, np.float32) if y_zero else rng.standard_normal(ny).astype(np.float32)
        m["dy"] = flh.DeviceBuffer.from_array(m["y0"], gpu)
    # ACT_Q8 of each column, then (for the column's first user with nx == 1)
    # that matrix's first tile right behind it
    placed = set()
    for p in order:
        tasks.append(mk(flh, T.ACT_Q8, x=dx.ptr + 4 * p * st, y=dx.ptr + 4 * p * st + flh.xq_offset(cols),
                        rows=cols // 32, cols=cols))

    def tile(m, r0, r1):
        rb = row_bytes(m["fmt"], cols)
        kw = dict(fmt=m["fmt"], x=dx.ptr + 4 * m["p0"] * st, y=m["dy"].ptr + 4 * r0, rows=r1 - r0, cols=cols,
                  nx=m["nx"], xstride=st, ystride=m["rows"], w_bytes=(r1 - r0) * rb)
        if m["idx"]:
            return mk(flh, T.STREAM_DOT_IDX, w=m["dw"].ptr + r0 * rb, aux=m["slot"].ptr, aux2=m["rows"] * rb, **kw)
        return mk(flh, T.STREAM_DOT, w=m["dw"].ptr + r0 * rb, **kw)
    # the last ACT_Q8's column: its first one-column, plain user goes right after it
    last = order[-1]
    for m in mats:
        if m["p0"] == last and m["nx"] == 1 and not m["idx"]:
            tasks.append(tile(m, *m["tiles"][0]))
            placed.add((id(m), 0))
            break
    for m in mats:
        for k, (r0, r1) in enumerate(m["tiles"]):
            if (id(m), k) not in placed:
                tasks.append(tile(m, r0, r1))
    tasks.append(mk(flh, T.SIGNAL))
    return dict(cols=cols, st=st, xs=xs, dx=dx, mats=mats, tasks=tasks)


def expected(orc, d):
    cols, st = d["cols"], d["st"]
    xq = orc.act_q8_cols(d["xs"], st)
    out = []
    for m in d["mats"]:
        rb = row_bytes(m["fmt"], cols)
        want = m["y0"].copy()
        off = 2 * m["rows"] * rb if m["idx"] else 0
        orc.stream_dot(m["fmt"], m["w"][off:off + m["rows"] * rb], m["rows"], cols, xq[m["p0"] * st:], want,
                       nx=m["nx"], xstride=st, ystride=m["rows"], i8_mask=I8_ALL, threads=8)
        out.append(want)
    return out


def read(d, gpu):
    return [m["dy"].download(np.float32, m["y0"].size, gpu) for m in d["mats"]]


@pytest.mark.parametrize("seed", CASES)
def test_random_task_table_bitwise(flh, orc, gpu, seed):
    d = build(flh, gpu, seed)
    print("[case] random table", seed, d["cols"], [(m["fmt"], m["rows"], m["nx"], len(m["tiles"]), m["idx"])
                                                    for m in d["mats"]], flush=True)
    flh.exec_tasks(d["tasks"], gpu, i8_mask=I8_ALL)
    for m, got, want in zip(d["mats"], read(d, gpu), expected(orc, d)):
        assert np.array_equal(bits(got), bits(want)), (m["fmt"], m["rows"], m["nx"], m["tiles"], m["idx"])


@pytest.mark.parametrize("seed", range(8))
def test_random_task_table_graph_replays(flh, orc, gpu, seed):
    """The table and the zeroing of its outputs captured in one HIP graph and
    replayed four times with eager work in between: every replay gives the
    oracle's bits (no memset nodes: outputs are cleared by a fill kernel)."""
    d = build(flh, gpu, 100 + seed, y_zero=True)
    print("[case] random table graph", seed, d["cols"], len(d["tasks"]), flush=True)
    want = expected(orc, d)
    with flh.Graph.capture(gpu) as g:
        for m in d["mats"]:
            m["dy"].zero(gpu)
        flh.exec_tasks(d["tasks"], gpu, i8_mask=I8_ALL)
    for rep in range(4):
        g.launch()
        gpu.sync()
        for m, got, w in zip(d["mats"], read(d, gpu), want):
            assert np.array_equal(bits(got), bits(w)), (rep, m["fmt"], m["rows"], m["nx"], m["idx"])
        for m in d["mats"]:                      # eager work between replays
            m["dy"].zero(gpu)
        gpu.sync()
    g.close()
