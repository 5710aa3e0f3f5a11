"""GPU parity at every BASELINE shape, full size, against the reference's own
compiled CPU code (oracle/_ref, built from the reference's sources and
shipped with the tree), run in the same process on the host cores.

Random weight blocks with sane fp16 scales (the reference tests' recipe),
activations N(0,1) with 1 % x20 outliers; the activation appendices are the
reference's ACT_Q8 (fl_exec_act_q8) and must equal the device's byte for
byte; the dots go through exec_task_cpu with the CPU default masks (the
int8 dots, src/runtime/quants.h:438-594) and must equal the device's bit for
bit.  Shapes: configs 0-4 of BASELINE.json at their real sizes (Q8_0
4096x4096 and the 14336-wide two-halves case, the four Q4_K layer shapes
unfused and with ACT_Q8 fused in, Q6_K vocab 128256x4096 and down, verify
N = 2 / 4 / 8 at both shapes, routed / grouped MoE expert dots at the
Mixtral expert shapes for batch 1 and 8)."""
import os

import numpy as np
import pytest

from oracle import Oracle, REF_SO, Q8_0, Q4_K, Q6_K, col_stride_floats, row_bytes, x_alloc_bytes
from util import sane_rows, activations
from test_gpu_parity import bits, say

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not os.path.exists(REF_SO), reason="oracle/_ref not built")]


@pytest.fixture(scope="module")
def ref():
    return Oracle(ref=True)


def ref_cols(ref, xs, st):
    """nx columns at stride st floats with the reference's ACT_Q8 appendices."""
    nx, cols = xs.shape
    buf = np.zeros(nx * st, dtype=np.float32)
    for p in range(nx):
        col = ref.act_q8(xs[p])
        buf[p * st:p * st + col.size // 4] = col.view(np.float32)
    return buf


def device_dot(flh, gpu, fmt, w, rows, cols, xs, st, fused=False):
    nx = xs.shape[0]
    hx = np.zeros(nx * st, dtype=np.float32)
    for p in range(nx):
        hx[p * st:p * st + cols] = xs[p]
    dx = flh.DeviceBuffer.from_array(hx, gpu)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    dy = flh.DeviceBuffer(nx * rows * 4)
    dy.zero(gpu)
    if fused:
        flh.act_q8_stream_dot(fmt, dw, rows, cols, dx, dy, gpu)
    else:
        flh.act_q8(dx, cols, gpu, nx=nx, xstride=st)
        flh.stream_dot(fmt, dw, rows, cols, dx, dy, gpu, nx=nx, xstride=st, ystride=rows)
    return dx.download(np.float32, nx * st, gpu), dy.download(np.float32, nx * rows, gpu)


CASES = [
    (Q8_0, 4096, 4096, 1, False), (Q8_0, 4096, 14336, 1, False),
    (Q4_K, 6144, 4096, 1, False), (Q4_K, 6144, 4096, 1, True),
    (Q4_K, 4096, 4096, 1, False), (Q4_K, 4096, 4096, 1, True),
    (Q4_K, 28672, 4096, 1, False), (Q4_K, 28672, 4096, 1, True),
    (Q4_K, 4096, 14336, 1, False),
    (Q6_K, 128256, 4096, 1, False), (Q6_K, 4096, 14336, 1, False),
    (Q4_K, 14336, 4096, 2, False), (Q4_K, 14336, 4096, 4, False), (Q4_K, 14336, 4096, 8, False),
    (Q4_K, 4096, 14336, 2, False), (Q4_K, 4096, 14336, 4, False), (Q4_K, 4096, 14336, 8, False),
]


@pytest.mark.parametrize("fmt,rows,cols,nx,fused", CASES)
def test_full_shape_equals_reference(flh, gpu, ref, fmt, rows, cols, nx, fused):
    say("full ref", fmt, rows, cols, nx, "fused" if fused else "")
    rng = np.random.default_rng(rows * 7 + cols + nx + fused)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    st = col_stride_floats(cols)
    gx, gy = device_dot(flh, gpu, fmt, w, rows, cols, xs, st, fused)
    rx = ref_cols(ref, xs, st)
    n8 = x_alloc_bytes(cols) // 4
    for p in range(nx):
        assert np.array_equal(bits(gx[p * st:p * st + n8]), bits(rx[p * st:p * st + n8])), f"appendix of column {p}"
    want = np.zeros(nx * rows, dtype=np.float32)
    ref.stream_dot(fmt, w, rows, cols, rx, want, nx=nx, xstride=st, ystride=rows, threads=16)
    assert np.array_equal(bits(gy), bits(want))


@pytest.mark.parametrize("ntok", [1, 8])
def test_moe_full_expert_shape_equals_reference(flh, gpu, ref, ntok):
    """Routed (batch 1) and grouped (batch 8) expert dots at the Mixtral expert
    shapes, gate/up 28672x4096 and down 4096x14336, 4 experts top 2: every
    (token, slot) pair's output equals the reference's STREAM_DOT_IDX tile
    (fl_idx_w, runtime_internal.h:149-152) on that pair's expert, bitwise."""
    E, K = 4, 2
    for rows, cols in ((28672, 4096), (4096, 14336)):
        say("full ref moe", ntok, rows, cols)
        rng = np.random.default_rng(ntok * 100 + cols)
        rb = rows * row_bytes(Q4_K, cols)
        w = sane_rows(Q4_K, E * rows, cols, rng)
        xs = activations(ntok, cols, rng, outliers=True)
        st = col_stride_floats(cols)
        ids = np.array([rng.permutation(E)[:K] for _ in range(ntok)], dtype=np.uint32).reshape(-1)
        rx = ref_cols(ref, xs, st)
        dx = flh.DeviceBuffer.from_array(rx, gpu)
        dw = flh.DeviceBuffer.from_array(w, gpu)
        did = flh.DeviceBuffer.from_array(ids, gpu)
        dy = flh.DeviceBuffer(ntok * K * rows * 4)
        dy.zero(gpu)
        flh.moe_dot(Q4_K, dw, rb, rows, cols, did, ntok, K, E, dx, st, False, dy, rows, gpu)
        got = dy.download(np.float32, ntok * K * rows, gpu)
        for p in range(ntok * K):
            t = p // K
            want = np.zeros(rows, dtype=np.float32)
            ref.stream_dot(Q4_K, w, rows, cols, rx[t * st:(t + 1) * st], want, id_slot=int(ids[p]), estride=rb)
            assert np.array_equal(bits(got[p * rows:(p + 1) * rows]), bits(want)), f"pair {p} expert {ids[p]}"
