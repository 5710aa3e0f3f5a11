"""RMSNORM -> ACT_Q8 on the device (flh_rmsnorm_act_q8, and RMSNORM + ACT_Q8
task pairs in flh_exec_tasks) against the oracle's fl_op_rmsnorm
(src/runtime/decode_params.h:101-106; oracle pinned to the reference's
own outputs in tests/test_oracle_norm.py), and the decoder's whole
norm -> quant -> matvec chain (src/model/decoder.cpp:874-880) against the
reference's chain (tests/golden/golden_norm.npz, and oracle/_ref at the
Llama-3-8B QKV and gate/up shapes) within 1e-3 * max|y|, the north-star
tolerance.

Bar: the reference sums the squares strictly in order on the CPU; the kernel
sums them as a tree, so y may differ from the reference by the rounding of
that sum: |y - y_ref| <= n * 2^-24 * |y_ref| + 2 ulp (the worst-case relative
error of an n-term sequential float sum, which bounds both orders).  Every
step after the sum is the reference's arithmetic, and the fused quantisation
is exact: the appendices equal ACT_Q8 of the y the kernel stored, byte for
byte; a STREAM_DOT of them equals the oracle's bit for bit."""
import ctypes

import numpy as np
import pytest

from oracle import Q4_K, col_stride_floats, x_alloc_bytes
from util import sane_rows, tuned

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def check_y(y, want, n):
    ulp = np.spacing(np.abs(want).astype(np.float32))
    assert np.all(np.abs(y - want) <= n * 2.0 ** -24 * np.abs(want) + 2 * ulp)


@pytest.mark.parametrize("n", [256, 768, 4096, 5120, 14336])
def test_rmsnorm_act_q8(flh, orc, gpu, n):
    print("[case] rmsnorm", n, flush=True)
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    st = col_stride_floats(n)
    dx = flh.DeviceBuffer.from_array(x, gpu)
    dw = flh.DeviceBuffer.from_array(wn, gpu)
    dy = flh.DeviceBuffer.from_array(np.zeros(st, np.float32), gpu)
    flh.rmsnorm_act_q8(dx, dw, dy, n, 1e-5, gpu)
    yb = dy.download(np.float32, st, gpu)
    y = yb[:n].copy()
    check_y(y, orc.rmsnorm(x, wn, 1e-5), n)
    nb = x_alloc_bytes(n)
    assert np.array_equal(yb.view(np.uint8)[:nb], orc.act_q8(y)[:nb]), "appendices == ACT_Q8(y)"


def test_rmsnorm_task_pair_fuses(flh, orc, gpu):
    """RMSNORM, ACT_Q8 of its output, a Q4_K STREAM_DOT of it: the table gives
    the bits of flh_rmsnorm_act_q8 followed by flh_stream_dot, and the dot
    equals the oracle's on the quantised y."""
    n, rows = 4096, 300
    rng = np.random.default_rng(5)
    x = rng.standard_normal(n).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    w = sane_rows(Q4_K, rows, n, rng)
    st = col_stride_floats(n)
    dx = flh.DeviceBuffer.from_array(x, gpu)
    dwn = flh.DeviceBuffer.from_array(wn, gpu)
    dy = flh.DeviceBuffer.from_array(np.zeros(st, np.float32), gpu)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    out = flh.DeviceBuffer.from_array(np.zeros(rows, np.float32), gpu)
    p = flh.RmsNormP(dwn.ptr, dx.ptr, dy.ptr, 1e-5, n)
    T = flh.TaskKind
    t0 = flh.Task(); t0.kind = int(T.RMSNORM); t0.aux = ctypes.addressof(p)
    t1 = flh.Task(); t1.kind = int(T.ACT_Q8); t1.x = dy.ptr; t1.y = dy.ptr + flh.xq_offset(n); t1.rows = n // 32
    t1.cols = n
    t2 = flh.Task(); t2.kind = int(T.STREAM_DOT); t2.fmt = Q4_K; t2.w = dw.ptr; t2.w_bytes = w.size; t2.x = dy.ptr
    t2.y = out.ptr; t2.rows = rows; t2.cols = n
    flh.exec_tasks([t0, t1, t2], gpu)
    yb = dy.download(np.float32, st, gpu)
    got = out.download(np.float32, rows, gpu)
    check_y(yb[:n], orc.rmsnorm(x, wn, 1e-5), n)
    want = np.zeros(rows, np.float32)
    orc.stream_dot(Q4_K, w, rows, n, yb, want)
    assert np.array_equal(bits(got), bits(want))
    # the same through the direct entry points
    dy2 = flh.DeviceBuffer.from_array(np.zeros(st, np.float32), gpu)
    flh.rmsnorm_act_q8(dx, dwn, dy2, n, 1e-5, gpu)
    assert np.array_equal(bits(dy2.download(np.float32, st, gpu)), bits(yb))


@pytest.mark.parametrize("cfg", ["1", "1,4", "1,8,1,5,2"])
@pytest.mark.parametrize("rows,n", [(5, 256), (9, 1024), (50, 2048), (300, 4096), (6144, 4096), (28672, 4096),
                                    (77, 8192), (33, 14336),
                                    # 20 superblocks: the 8-wave plan needs exactly all of a
                                    # workgroup's LDS, with no room for the prologue's static
                                    # norm partials (the launcher now plans around them)
                                    (9180, 5120)])
def test_rmsnorm_stream_dot(flh, orc, gpu, cfg, rows, n):
    """RMSNORM -> ACT_Q8 -> Q4_K dot in one launch (flh_rmsnorm_stream_dot;
    14336 columns take the two-launch path): the normalised column, its
    appendices and y += W xn equal rmsnorm_act_q8 followed by stream_dot bit
    for bit, y is within the sequential-sum bound of the reference, and the
    dot equals the oracle's on the stored column."""
    print("[case] rmsnorm dot", cfg, rows, n, flush=True)
    rng = np.random.default_rng(rows + n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    w = sane_rows(Q4_K, rows, n, rng)
    y0 = rng.standard_normal(rows).astype(np.float32)
    st = col_stride_floats(n)
    dx = flh.DeviceBuffer.from_array(x, gpu)
    dwn = flh.DeviceBuffer.from_array(wn, gpu)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    outs = []
    for fused in (True, False):
        dxn = flh.DeviceBuffer.from_array(np.zeros(st, np.float32), gpu)
        dy = flh.DeviceBuffer.from_array(y0, gpu)
        with tuned(flh, FLH_SBL=cfg):
            if fused:
                flh.rmsnorm_stream_dot(Q4_K, dw, rows, n, dx, dwn, 1e-5, dxn, dy, gpu)
            else:
                flh.rmsnorm_act_q8(dx, dwn, dxn, n, 1e-5, gpu)
                flh.stream_dot(Q4_K, dw, rows, n, dxn, dy, gpu)
        outs.append((dxn.download(np.float32, st, gpu), dy.download(np.float32, rows, gpu)))
    (xa, ya), (xb, yb) = outs
    assert np.array_equal(bits(xa), bits(xb)), "normalised column and appendices"
    assert np.array_equal(bits(ya), bits(yb)), "dot"
    check_y(xa[:n], orc.rmsnorm(x, wn, 1e-5), n)
    want = y0.copy()
    orc.stream_dot(Q4_K, w, rows, n, xa, want)
    assert np.array_equal(bits(ya), bits(want))


@pytest.mark.parametrize("fmt", [1, 4])          # Q8_0, Q6_K: the two-launch path
def test_rmsnorm_stream_dot_other_formats(flh, orc, gpu, fmt):
    """Formats the one-launch kernel does not take give the separate calls' bits."""
    print("[case] rmsnorm dot fmt", fmt, flush=True)
    rows, n = 200, 4096
    rng = np.random.default_rng(fmt)
    x = rng.standard_normal(n).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    w = sane_rows(fmt, rows, n, rng)
    st = col_stride_floats(n)
    dx, dwn, dw = (flh.DeviceBuffer.from_array(a, gpu) for a in (x, wn, w))
    outs = []
    for fused in (True, False):
        dxn = flh.DeviceBuffer.from_array(np.zeros(st, np.float32), gpu)
        dy = flh.DeviceBuffer.from_array(np.zeros(rows, np.float32), gpu)
        if fused:
            flh.rmsnorm_stream_dot(fmt, dw, rows, n, dx, dwn, 1e-5, dxn, dy, gpu)
        else:
            flh.rmsnorm_act_q8(dx, dwn, dxn, n, 1e-5, gpu)
            flh.stream_dot(fmt, dw, rows, n, dxn, dy, gpu)
        outs.append((dxn.download(np.float32, st, gpu), dy.download(np.float32, rows, gpu)))
    assert np.array_equal(bits(outs[0][0]), bits(outs[1][0]))
    assert np.array_equal(bits(outs[0][1]), bits(outs[1][1]))


def test_rmsnorm_stream_dot_rejects_overlap(flh, gpu):
    """xn overlapping x is an argument error (the launch would read x while
    other workgroups write y); nothing is launched."""
    n, rows = 4096, 16
    st = col_stride_floats(n)
    buf = flh.DeviceBuffer.from_array(np.ones(2 * st, np.float32), gpu)
    wn = flh.DeviceBuffer.from_array(np.ones(n, np.float32), gpu)
    w = flh.DeviceBuffer.from_array(sane_rows(Q4_K, rows, n, np.random.default_rng(0)), gpu)
    y = flh.DeviceBuffer.from_array(np.zeros(rows, np.float32), gpu)
    with pytest.raises(flh.FlhError):
        flh.rmsnorm_stream_dot(Q4_K, w, rows, n, buf, wn, 1e-5, buf.ptr + 1024, y, gpu)


def test_rmsnorm_dot_triple_in_graph(flh, orc, gpu):
    """RMSNORM + ACT_Q8 + STREAM_DOT in a HIP graph: every replay (with eager
    work and synchronisations in between) gives the eager run's bits."""
    n, rows = 4096, 6144
    rng = np.random.default_rng(21)
    x = rng.standard_normal(n).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    w = sane_rows(Q4_K, rows, n, rng)
    st = col_stride_floats(n)
    dx, dwn, dw = (flh.DeviceBuffer.from_array(a, gpu) for a in (x, wn, w))
    dxn = flh.DeviceBuffer.from_array(np.zeros(st, np.float32), gpu)
    dy = flh.DeviceBuffer.from_array(np.zeros(rows, np.float32), gpu)
    p = flh.RmsNormP(dwn.ptr, dx.ptr, dxn.ptr, 1e-5, n)
    T = flh.TaskKind
    t0 = flh.Task(); t0.kind = int(T.RMSNORM); t0.aux = ctypes.addressof(p)
    t1 = flh.Task(); t1.kind = int(T.ACT_Q8); t1.x = dxn.ptr; t1.y = dxn.ptr + flh.xq_offset(n); t1.rows = n // 32
    t1.cols = n
    t2 = flh.Task(); t2.kind = int(T.STREAM_DOT); t2.fmt = Q4_K; t2.w = dw.ptr; t2.w_bytes = w.size; t2.x = dxn.ptr
    t2.y = dy.ptr; t2.rows = rows; t2.cols = n
    tasks = [t0, t1, t2]
    flh.exec_tasks(tasks, gpu)
    ref = dy.download(np.float32, rows, gpu).copy()
    refx = dxn.download(np.float32, st, gpu).copy()
    with flh.Graph.capture(gpu) as g:
        flh.exec_tasks(tasks, gpu)
    for k in range(3):
        dy.zero(gpu)
        g.launch()
        gpu.sync()
        assert np.array_equal(bits(dy.download(np.float32, rows, gpu)), bits(ref)), k
        assert np.array_equal(bits(dxn.download(np.float32, st, gpu)), bits(refx)), k
    g.close()


@pytest.mark.parametrize("cfg", ["1", "0"])
@pytest.mark.parametrize("rows,n", [(20480, 4096), (28672, 4096), (300, 4096), (77, 8192)])
def test_rmsnorm_stream_dot_kernels_agree(flh, orc, gpu, cfg, rows, n):
    """Above 2^18 superblocks (and with FLH_SBL=0 at any size) the one-launch
    RMSNORM -> dot runs on the four-lanes-per-superblock kernel: same bits as
    the separate launches there too."""
    print("[case] rmsnorm dot kernels", cfg, rows, n, flush=True)
    rng = np.random.default_rng(rows + 3 * n)
    x = (rng.standard_normal(n) * 2).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    w = sane_rows(Q4_K, rows, n, rng)
    y0 = rng.standard_normal(rows).astype(np.float32)
    st = col_stride_floats(n)
    dx, dwn, dw = (flh.DeviceBuffer.from_array(a, gpu) for a in (x, wn, w))
    outs = []
    for fused in (True, False):
        dxn = flh.DeviceBuffer.from_array(np.zeros(st, np.float32), gpu)
        dy = flh.DeviceBuffer.from_array(y0, gpu)
        with tuned(flh, FLH_SBL=cfg):
            if fused:
                flh.rmsnorm_stream_dot(Q4_K, dw, rows, n, dx, dwn, 1e-5, dxn, dy, gpu)
            else:
                flh.rmsnorm_act_q8(dx, dwn, dxn, n, 1e-5, gpu)
                flh.stream_dot(Q4_K, dw, rows, n, dxn, dy, gpu)
        outs.append((dxn.download(np.float32, st, gpu), dy.download(np.float32, rows, gpu)))
    assert np.array_equal(bits(outs[0][0]), bits(outs[1][0]))
    assert np.array_equal(bits(outs[0][1]), bits(outs[1][1]))
    want = y0.copy()
    orc.stream_dot(Q4_K, w, rows, n, outs[0][0], want, threads=8)
    assert np.array_equal(bits(outs[0][1]), bits(want))


def test_param_blocks_device_memory_rejected(flh, orc, gpu):
    """Decode-op param blocks are read by the host when the table is issued:
    a block in device memory (where a binding that put everything in the
    device arena would place it) is rejected with FLH_ERR_ARG before any
    launch; the same block in pinned host memory (flh_host_alloc, where the
    binding's aux_alloc puts it) runs the chain with the bits of a block in
    ordinary host memory."""
    print("[case] param block placement", flush=True)
    n, rows = 4096, 64
    rng = np.random.default_rng(6)
    x = rng.standard_normal(n).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    w = sane_rows(Q4_K, rows, n, rng)
    st = col_stride_floats(n)
    dx = flh.DeviceBuffer.from_array(x, gpu)
    dwn = flh.DeviceBuffer.from_array(wn, gpu)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    T = flh.TaskKind

    def run(aux_of):
        dy = flh.DeviceBuffer.from_array(np.zeros(st, np.float32), gpu)
        out = flh.DeviceBuffer.from_array(np.zeros(rows, np.float32), gpu)
        p = flh.RmsNormP(dwn.ptr, dx.ptr, dy.ptr, 1e-5, n)
        t0 = flh.Task(); t0.kind = int(T.RMSNORM); t0.aux = aux_of(p)
        t1 = flh.Task(); t1.kind = int(T.ACT_Q8); t1.x = dy.ptr; t1.y = dy.ptr + flh.xq_offset(n)
        t1.rows = n // 32; t1.cols = n
        t2 = flh.Task(); t2.kind = int(T.STREAM_DOT); t2.fmt = Q4_K; t2.w = dw.ptr; t2.w_bytes = w.size
        t2.x = dy.ptr; t2.y = out.ptr; t2.rows = rows; t2.cols = n
        flh.exec_tasks([t0, t1, t2], gpu)
        return dy.download(np.float32, st, gpu), out.download(np.float32, rows, gpu)

    keep = []

    def on_device(p):
        b = flh.DeviceBuffer.from_array(np.frombuffer(bytes(p), np.uint8), gpu)
        keep.append(b)
        return b.ptr

    def pinned(p):
        h = flh.HostBuffer(ctypes.sizeof(p))
        ctypes.memmove(h.ptr, ctypes.addressof(p), ctypes.sizeof(p))
        keep.append(h)
        return h.ptr

    with pytest.raises(flh.FlhError) as e:
        run(on_device)
    assert e.value.code == flh.ERR_ARG and "param block" in str(e.value)
    gpu.sync()
    want = run(lambda p: keep.append(p) or ctypes.addressof(p))
    got = run(pinned)
    assert np.array_equal(bits(got[0]), bits(want[0])) and np.array_equal(bits(got[1]), bits(want[1]))


def norm_dot_device(flh, gpu, x, wn, w, rows, cols):
    """flh_rmsnorm_stream_dot: the normed column (with appendices) and y."""
    st = col_stride_floats(cols)
    dx = flh.DeviceBuffer.from_array(x, gpu)
    dwn = flh.DeviceBuffer.from_array(wn, gpu)
    dxn = flh.DeviceBuffer.from_array(np.zeros(st, np.float32), gpu)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    dy = flh.DeviceBuffer.from_array(np.zeros(rows, np.float32), gpu)
    flh.rmsnorm_stream_dot(Q4_K, dw, rows, cols, dx, dwn, 1e-5, dxn, dy, gpu)
    return dxn.download(np.uint8, x_alloc_bytes(cols), gpu), dy.download(np.float32, rows, gpu)


@pytest.mark.parametrize("i", [0, 1])
def test_norm_chain_vs_reference_golden(flh, gpu, i):
    """The device chain against the reference's own chain (golden vectors):
    the normed column within the sequential-sum bound, the dot within
    1e-3 * max|y_ref|."""
    from norm_cases import CHAIN_CASES, chain_inputs, digest
    import os
    G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_norm.npz"))
    rows, cols, seed = CHAIN_CASES[i]
    print("[case] norm chain golden", rows, cols, flush=True)
    x, wn, w = chain_inputs(rows, cols, seed)
    assert bytes(G[f"c{i}_digest"]) == digest(x, wn, w)
    col, y = norm_dot_device(flh, gpu, x, wn, w, rows, cols)
    want_col, want = G[f"c{i}_col"], G[f"c{i}_y"]
    check_y(col[:4 * cols].view(np.float32), want_col[:4 * cols].view(np.float32), cols)
    assert np.max(np.abs(y - want)) <= 1e-3 * np.max(np.abs(want))


@pytest.mark.parametrize("rows", [6144, 28672])
def test_norm_chain_vs_reference_full_shape(flh, gpu, rows):
    """At the Llama-3-8B QKV and gate/up shapes (one launch on the device):
    the reference's chain, run from its own compiled code (oracle/_ref; the
    pinned oracle where that library is absent), against
    flh_rmsnorm_stream_dot, within 1e-3 * max|y_ref|."""
    from oracle import Oracle, REF_SO
    import os
    cols = 4096
    print("[case] norm chain full", rows, cols, flush=True)
    rng = np.random.default_rng(rows)
    x = rng.standard_normal(cols).astype(np.float32)
    x[rng.random(cols) < 0.01] *= 20.0
    wn = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    w = sane_rows(Q4_K, rows, cols, rng)
    ref = Oracle(ref=os.path.exists(REF_SO))
    rcol = ref.act_q8(ref.rmsnorm(x, wn, 1e-5))
    want = np.zeros(rows, np.float32)
    ref.stream_dot(Q4_K, w, rows, cols, rcol.view(np.float32), want, threads=8)
    col, y = norm_dot_device(flh, gpu, x, wn, w, rows, cols)
    check_y(col[:4 * cols].view(np.float32), rcol[:4 * cols].view(np.float32), cols)
    assert np.max(np.abs(y - want)) <= 1e-3 * np.max(np.abs(want))
