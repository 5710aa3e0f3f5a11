"""The Task-table adapter (flh_exec_tasks) against the oracle.

A frozen graph's task table, in the reference's own Task layout
(include/fastllm/fastllm.h:65-97), is run through the C-ABI: ACT_Q8 +
consecutive STREAM_DOT row tiles (fused into one launch), a multi-column
tile, a STREAM_DOT_IDX tile, MERGE and SIGNAL, in the order run_serial walks
(src/runtime/graph.cpp:116-148).  Every output must equal the oracle's
exec_task_cpu result bit for bit; HIP-graph replays of the same table must
reproduce the eager result every time.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import Q4_K, Q6_K, Q8_0, col_stride_floats, row_bytes
from util import sane_rows, activations

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def mk(flh, kind, **kw):
    t = flh.Task()
    t.kind = int(kind)
    for k, v in kw.items():
        setattr(t, k, v)
    return t


def build(flh, gpu, rng, cols=1024):
    st = col_stride_floats(cols)
    xs = activations(2, cols, rng, outliers=True)
    xb = np.zeros(2 * st, dtype=np.float32)
    xb[:cols], xb[st:st + cols] = xs[0], xs[1]
    d = {"cols": cols, "st": st, "xs": xs}
    d["x"] = flh.DeviceBuffer.from_array(xb, gpu)
    d["w4"] = sane_rows(Q4_K, 600, cols, rng)
    d["w6"] = sane_rows(Q6_K, 3 * 40, cols, rng)
    d["w8"] = sane_rows(Q8_0, 70, cols, rng)
    for k in ("w4", "w6", "w8"):
        d["d" + k] = flh.DeviceBuffer.from_array(d[k], gpu)
    d["slot"] = flh.DeviceBuffer.from_array(np.array([2], dtype=np.uint32), gpu)
    d["y4"] = flh.DeviceBuffer(600 * 4)
    d["y6"] = flh.DeviceBuffer(40 * 4)
    d["y8"] = flh.DeviceBuffer(2 * 70 * 4)
    d["parts"] = flh.DeviceBuffer(2 * 40 * 4)
    d["merged"] = flh.DeviceBuffer(40 * 4)
    return d


def table(flh, d):
    x0, x1 = d["x"].ptr, d["x"].ptr + 4 * d["st"]
    cols, st = d["cols"], d["st"]
    rb4, rb6, rb8 = row_bytes(Q4_K, cols), row_bytes(Q6_K, cols), row_bytes(Q8_0, cols)
    T = flh.TaskKind
    # ACT_Q8(x0) directly precedes its first Q4_K tile, so the adapter fuses
    # that pair; the later tiles (and the Q8_0 tile's q8_1 reads) then depend
    # on the appendix the fused kernel wrote.
    t = [mk(flh, T.ACT_Q8, x=x1, y=x1 + flh.xq_offset(cols), rows=cols // 32, cols=cols),
         mk(flh, T.ACT_Q8, x=x0, y=x0 + flh.xq_offset(cols), rows=cols // 32, cols=cols)]
    # Q4_K matrix in three row tiles
    r0 = 0
    for n in (256, 256, 88):
        t.append(mk(flh, T.STREAM_DOT, fmt=Q4_K, w=d["dw4"].ptr + r0 * rb4, w_bytes=n * rb4, x=x0,
                    y=d["y4"].ptr + 4 * r0, rows=n, cols=cols))
        r0 += n
    # Q6_K expert 2 of 3 via the id slot
    t.append(mk(flh, T.STREAM_DOT_IDX, fmt=Q6_K, w=d["dw6"].ptr, w_bytes=40 * rb6, x=x1, y=d["y6"].ptr,
                rows=40, cols=cols, aux=d["slot"].ptr, aux2=40 * rb6))
    # Q8_0 two-column tile
    t.append(mk(flh, T.STREAM_DOT, fmt=Q8_0, w=d["dw8"].ptr, w_bytes=70 * rb8, x=x0, y=d["y8"].ptr,
                rows=70, cols=cols, nx=2, xstride=st, ystride=70))
    # two partial slots of the Q6_K expert rows, then MERGE, then SIGNAL
    for p in range(2):
        t.append(mk(flh, T.STREAM_DOT, fmt=Q6_K, w=d["dw6"].ptr + 40 * rb6 * p, w_bytes=40 * rb6,
                    x=x0 if p == 0 else x1, y=d["parts"].ptr + 4 * 40 * p, rows=40, cols=cols))
    t.append(mk(flh, T.MERGE, x=d["parts"].ptr, y=d["merged"].ptr, rows=40, cols=2))
    t.append(mk(flh, T.SIGNAL))
    return t


def expected(orc, d):
    cols, st = d["cols"], d["st"]
    xq = orc.act_q8_cols(d["xs"], st)
    x0, x1 = xq[:st], xq[st:]
    y4 = np.zeros(600, np.float32)
    orc.stream_dot(Q4_K, d["w4"], 600, cols, x0, y4)
    y6 = np.zeros(40, np.float32)
    orc.stream_dot(Q6_K, d["w6"], 40, cols, x1, y6, id_slot=2, estride=40 * row_bytes(Q6_K, cols))
    y8 = np.zeros(140, np.float32)
    orc.stream_dot(Q8_0, d["w8"], 70, cols, xq, y8, nx=2, xstride=st, ystride=70)
    parts = np.zeros((2, 40), np.float32)
    for p in range(2):
        orc.stream_dot(Q6_K, d["w6"][40 * row_bytes(Q6_K, cols) * p:], 40, cols, x0 if p == 0 else x1, parts[p])
    # MERGE: acc = 0 + p0, then + p1 (runtime_internal.h:274-281)
    merged = np.array([np.float32(np.float32(0.0) + parts[0][i]) + parts[1][i] for i in range(40)],
                      dtype=np.float32)
    return y4, y6, y8, merged


def zero_outputs(d, gpu):
    for k in ("y4", "y6", "y8", "parts", "merged"):
        d[k].zero(gpu)


def read(d, gpu):
    return (d["y4"].download(np.float32, 600, gpu), d["y6"].download(np.float32, 40, gpu),
            d["y8"].download(np.float32, 140, gpu), d["merged"].download(np.float32, 40, gpu))


# 14336 columns: the ACT_Q8 is wider than the per-workgroup fusion takes, so
# it runs as a launch of its own ahead of the tiles
@pytest.mark.parametrize("cols", [1024, 14336])
def test_task_table_bitwise(flh, orc, gpu, cols):
    print("[case] task table eager", cols, flush=True)
    d = build(flh, gpu, np.random.default_rng(7), cols)
    zero_outputs(d, gpu)
    flh.exec_tasks(table(flh, d), gpu)
    for g, w in zip(read(d, gpu), expected(orc, d)):
        assert np.array_equal(bits(g), bits(w))


@pytest.mark.parametrize("cols", [1024, 14336])
def test_task_table_graph_replays(flh, orc, gpu, cols):
    """Capture the table (and the zeroing) once, replay it several times with
    eager work in between; every replay equals the eager result."""
    print("[case] task table graph", cols, flush=True)
    d = build(flh, gpu, np.random.default_rng(8), cols)
    want = expected(orc, d)
    tasks = table(flh, d)
    with flh.Graph.capture(gpu) as g:
        zero_outputs(d, gpu)
        flh.exec_tasks(tasks, gpu)
    for rep in range(4):
        g.launch()
        gpu.sync()
        for got, w in zip(read(d, gpu), want):
            assert np.array_equal(bits(got), bits(w)), rep
        zero_outputs(d, gpu)          # eager work between replays
        gpu.sync()
    g.close()


def test_unsupported_kind_launches_nothing(flh, gpu):
    d = build(flh, gpu, np.random.default_rng(9))
    zero_outputs(d, gpu)
    t = table(flh, d)
    t.insert(3, mk(flh, flh.TaskKind.ATTN_HEAD, aux=d["slot"].ptr))
    with pytest.raises(flh.FlhError) as e:
        flh.exec_tasks(t, gpu)
    assert e.value.code == flh.ERR_UNSUPPORTED
    gpu.sync()
    assert not np.any(d["y4"].download(np.float32, 600, gpu))


def test_masks_same_bits_every_entry_point(flh, orc, gpu):
    """Masks are used as given by every entry point.  With the reference's
    GPU-default masks (kernels.h:927-940: Q6_K off both int8 masks) the
    table's Q6_K tiles take the fp32 dequant route, as the oracle's
    exec_task_cpu does with those masks, and one Q6_K dot through the table
    equals the same dot through flh_stream_dot with the same masks, bit for
    bit; the other formats keep their int8 routes."""
    print("[case] task table gpu masks", flush=True)
    d = build(flh, gpu, np.random.default_rng(10), 1024)
    cols, st = d["cols"], d["st"]
    gpu_i8 = (1 << 1) | (1 << 2) | (1 << 3) | (1 << 5) | (1 << 6)
    gpu_i8k = 1 << 3
    zero_outputs(d, gpu)
    flh.exec_tasks(table(flh, d), gpu, i8_mask=gpu_i8, i8k_mask=gpu_i8k)
    y4, y6, y8, merged = read(d, gpu)
    xq = orc.act_q8_cols(d["xs"], st)
    x0, x1 = xq[:st], xq[st:]
    f6 = np.zeros(40, np.float32)
    orc.stream_dot(Q6_K, d["w6"], 40, cols, x1, f6, id_slot=2, estride=40 * row_bytes(Q6_K, cols),
                   i8_mask=gpu_i8, i8k_mask=gpu_i8k)
    assert np.array_equal(bits(y6), bits(f6))
    w4 = np.zeros(600, np.float32)
    orc.stream_dot(Q4_K, d["w4"], 600, cols, x0, w4, i8_mask=gpu_i8, i8k_mask=gpu_i8k)
    assert np.array_equal(bits(y4), bits(w4))
    # the same Q6_K expert dot through flh_stream_dot with the same masks
    rb6 = row_bytes(Q6_K, cols)
    dy = flh.DeviceBuffer(40 * 4)
    dy.zero(gpu)
    flh.stream_dot(Q6_K, d["dw6"].ptr + 2 * 40 * rb6, 40, cols, d["x"].ptr + 4 * st, dy, gpu,
                   i8_mask=gpu_i8, i8k_mask=gpu_i8k, w_bytes=40 * rb6)
    assert np.array_equal(bits(dy.download(np.float32, 40, gpu)), bits(y6))
    # and with the CPU-default masks both give the q8_K int8 bits
    zero_outputs(d, gpu)
    flh.exec_tasks(table(flh, d), gpu)
    dy.zero(gpu)
    flh.stream_dot(Q6_K, d["dw6"].ptr + 2 * 40 * rb6, 40, cols, d["x"].ptr + 4 * st, dy, gpu, w_bytes=40 * rb6)
    want = expected(orc, d)
    assert np.array_equal(bits(read(d, gpu)[1]), bits(want[1]))
    assert np.array_equal(bits(dy.download(np.float32, 40, gpu)), bits(want[1]))




def test_arena_alignment_and_exhaustion(flh, gpu):
    """flh_arena_alloc (Arena::alloc, src/runtime/arena.cpp:54-74): every
    pointer is aligned as an address to the requested power of two, blocks
    never overlap, and a request past the end (or one whose size would wrap)
    is FLH_ERR_NOMEM, leaving the arena usable."""
    a = flh.Arena(1 << 20)
    try:
        got = []
        for i, (n, al) in enumerate([(1, 16), (100, 4096), (3, 64), (5000, 65536), (7, 256)]):
            p = a.alloc(n, al)
            assert p % al == 0, (n, al)
            got.append((p, n))
        got.sort()
        for (p0, n0), (p1, _) in zip(got, got[1:]):
            assert p0 + n0 <= p1
        used = a.used
        for n in (1 << 21, (1 << 64) - 1):
            with pytest.raises(flh.FlhError) as e:
                a.alloc(n, 16)
            assert e.value.code == flh.ERR_NOMEM
        assert a.used == used
        with pytest.raises(flh.FlhError) as e:
            a.alloc(16, 48)
        assert e.value.code == flh.ERR_ARG
        assert a.alloc(16, 16) % 16 == 0
    finally:
        a.close()
