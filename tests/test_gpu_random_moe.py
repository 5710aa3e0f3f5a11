"""Seeded random grouped expert dots (flh_moe_dot, flh_router_moe_dot),
bitwise against the oracle's per-pair STREAM_DOT_IDX tiles.

Each case draws the format (Q4_K, Q6_K, Q8_0, Q5_0, IQ2_XXS, IQ3_XXS), the
expert count (2-16), top-k (1-4), the token batch (1-16), the expert shape,
per-slot or per-token activations, old y and the routing (ids given, or the
router fused into the launch with the reference's top-k and softmax), so the
launcher's choices between the routed one-token kernel, the matrix-core and
streaming grouped kernels, the register fallback and the per-pair tiles (the
32-weight-block formats beyond the routed launch's plan) all get random
inputs.
Every (token, slot) pair's y must equal exec_task_cpu's STREAM_DOT_IDX tile
for its expert (src/runtime/runtime_internal.h:149-152, src/model/decoder.cpp:
941-996), bit for bit; fused routing must give the oracle router's ids
(fl_op_router_sel, src/runtime/decode_params.h:234-265).
"""
import numpy as np
import pytest

from oracle import Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS, col_stride_floats, row_bytes
from util import sane_rows, activations
from test_gpu_moe import route, bits, say

pytestmark = pytest.mark.gpu

FMTS = [Q4_K, Q4_K, Q4_K, Q6_K, Q6_K, Q8_0, Q5_0, IQ2_XXS, IQ3_XXS]


def make_cases(n=40, seed=77):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        fmt = int(FMTS[rng.integers(len(FMTS))])
        E = int(rng.integers(2, 17))
        K = int(rng.integers(1, min(E, 4) + 1))
        ntok = int(rng.integers(1, 17)) if rng.random() < 0.7 else 1
        if fmt in (IQ2_XXS, IQ3_XXS):
            cols = 2048 * int(rng.integers(1, 5)) if rng.random() < 0.6 else 256 * int(rng.integers(1, 40))
        elif fmt in (Q8_0, Q5_0):
            cols = 256 * int(rng.integers(1, 65))
        else:
            cols = 256 * int(rng.integers(1, 57))
        rows = int(rng.integers(1, 1500))
        while rows * cols * E > 60_000_000:
            rows = max(1, rows // 2)
        per_slot = bool(rng.random() < 0.4)
        fused = bool(rng.random() < 0.4)
        out.append((i, fmt, E, K, ntok, rows, cols, per_slot, fused))
    return out


@pytest.mark.parametrize("i,fmt,E,K,ntok,rows,cols,per_slot,fused", make_cases())
def test_random_grouped_expert_dot(flh, orc, gpu, i, fmt, E, K, ntok, rows, cols, per_slot, fused):
    say("random moe", i, fmt, E, K, ntok, rows, cols, per_slot, fused)
    rng = np.random.default_rng(500 + i)
    logits, ids, _ = route(orc, ntok, E, K, rng)
    rb = row_bytes(fmt, cols)
    estride = rows * rb
    w = sane_rows(fmt, rows * E, cols, rng)
    nx = ntok * K if per_slot else ntok
    xs = activations(nx, cols, rng, outliers=True)
    st = col_stride_floats(cols)
    buf = np.zeros(nx * st, dtype=np.float32)
    for p in range(nx):
        buf[p * st:p * st + cols] = xs[p]
    dx = flh.DeviceBuffer.from_array(buf, gpu)
    flh.act_q8(dx, cols, gpu, nx=nx, xstride=st)
    ref_x = orc.act_q8_cols(xs, st)
    y0 = rng.standard_normal(ntok * K * rows).astype(np.float32)
    dy = flh.DeviceBuffer.from_array(y0, gpu)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    if fused:
        dl = flh.DeviceBuffer.from_array(logits, gpu)
        di, dg = flh.DeviceBuffer(4 * ntok * K), flh.DeviceBuffer(4 * ntok * K)
        flh.router_moe_dot(fmt, dw, estride, rows, cols, dl, ntok, E, K, 1, 1.0, di, dg, dx, st, per_slot, dy, rows,
                           gpu)
        assert np.array_equal(di.download(np.uint32, ntok * K, gpu), ids.ravel())
    else:
        di = flh.DeviceBuffer.from_array(ids.ravel(), gpu)
        flh.moe_dot(fmt, dw, estride, rows, cols, di, ntok, K, E, dx, st, per_slot, dy, rows, gpu)
    got = dy.download(np.float32, y0.size, gpu)
    want = y0.copy()
    i8 = 0b11110 | (1 << IQ2_XXS) | (1 << IQ3_XXS)
    for t in range(ntok):
        for k in range(K):
            j = t * K + k
            xi = j if per_slot else t
            yi = want[j * rows:(j + 1) * rows]
            orc.stream_dot(fmt, w, rows, cols, ref_x[xi * st:(xi + 1) * st], yi, id_slot=int(ids[t, k]),
                           estride=estride, i8_mask=i8, threads=8)
            want[j * rows:(j + 1) * rows] = yi
    assert np.array_equal(bits(got), bits(want))
