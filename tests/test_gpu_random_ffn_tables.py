"""Seeded random one-token MoE FFN task tables through flh_exec_tasks.

Each table is the reference decoder's expert FFN (src/model/decoder.cpp:
874-880, 941-996): RMSNORM, ACT_Q8 (optionally a dense "shared" STREAM_DOT
right behind it, so the adapter runs the norm -> quant -> dot triple in one
launch), ROUTER_SEL, per routed slot the gate/up STREAM_DOT_IDX cut into
random row tiles, SILU_MUL + ACT_Q8 (one fused launch), the down
STREAM_DOT_IDX, then WMERGE with the residual, and SIGNAL; random widths,
expert counts, top-k and formats.  The op parameter blocks stay in host
memory, where the adapter reads them.

Each stage is checked against the oracle on the device's own input to that
stage: appendices byte for byte, ids equal, every dot bit for bit, WMERGE bit
for bit; within tolerance only where the reference sums in order on the CPU
(RMSNORM: the sequential-sum bound) or calls expf (gates rtol 2e-6, silu
rtol 4e-7).
"""
import ctypes as C

import numpy as np
import pytest

from oracle import Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, col_stride_floats, row_bytes, x_alloc_bytes
from util import sane_rows, activations
from test_gpu_tasks import mk, bits

pytestmark = pytest.mark.gpu

FMTS = [Q4_K, Q4_K, Q6_K, Q8_0, Q5_0, IQ2_XXS]
I8_ALL = 0b1111110


@pytest.mark.parametrize("seed", range(16))
def test_random_moe_ffn_table(flh, orc, gpu, seed):
    rng = np.random.default_rng(900 + seed)
    D = 256 * int(rng.integers(1, 17))
    FF = 256 * int(rng.integers(1, 17))
    E = int(rng.integers(2, 9))
    K = int(rng.integers(1, min(E, 4) + 1))
    fgu, fdn = int(FMTS[rng.integers(len(FMTS))]), int(FMTS[rng.integers(len(FMTS))])
    shared = bool(rng.random() < 0.5)
    norm = int(rng.integers(0, 2))
    print("[case] random ffn table", seed, D, FF, E, K, fgu, fdn, shared, norm, flush=True)
    T = flh.TaskKind
    stD, stF = col_stride_floats(D), col_stride_floats(FF)
    x = (rng.standard_normal(D) * 2).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    logits = rng.standard_normal(E).astype(np.float32)
    wgu = sane_rows(fgu, E * 2 * FF, D, rng)
    wdn = sane_rows(fdn, E * D, FF, rng)
    ws = sane_rows(Q4_K, FF, D, rng) if shared else None
    egu, edn = 2 * FF * row_bytes(fgu, D), D * row_bytes(fdn, FF)
    dx, dwn, dlog = (flh.DeviceBuffer.from_array(a, gpu) for a in (x, wn, logits))
    dxn = flh.DeviceBuffer.from_array(np.zeros(stD, np.float32), gpu)
    dgu_w, ddn_w = flh.DeviceBuffer.from_array(wgu, gpu), flh.DeviceBuffer.from_array(wdn, gpu)
    dids, dgates = flh.DeviceBuffer(4 * K), flh.DeviceBuffer(4 * K)
    dgu = flh.DeviceBuffer.from_array(np.zeros(K * 2 * FF, np.float32), gpu)
    dh = flh.DeviceBuffer.from_array(np.zeros(K * stF, np.float32), gpu)
    dparts = flh.DeviceBuffer.from_array(np.zeros(K * D, np.float32), gpu)
    dout = flh.DeviceBuffer(4 * D)
    if shared:
        dsw = flh.DeviceBuffer.from_array(ws, gpu)
        dsy = flh.DeviceBuffer.from_array(np.zeros(FF, np.float32), gpu)
    keep = []

    def host(p):
        keep.append(p)
        return C.addressof(p)

    tasks = [mk(flh, T.RMSNORM, aux=host(flh.RmsNormP(dwn.ptr, dx.ptr, dxn.ptr, 1e-5, D))),
             mk(flh, T.ACT_Q8, x=dxn.ptr, y=dxn.ptr + flh.xq_offset(D), rows=D // 32, cols=D)]
    if shared:
        tasks.append(mk(flh, T.STREAM_DOT, fmt=Q4_K, w=dsw.ptr, w_bytes=FF * row_bytes(Q4_K, D), x=dxn.ptr,
                        y=dsy.ptr, rows=FF, cols=D))
    tasks.append(mk(flh, T.ROUTER_SEL, aux=host(flh.RouterP(dlog.ptr, dids.ptr, dgates.ptr, E, K, norm, 1.0))))
    rbg, rbd = row_bytes(fgu, D), row_bytes(fdn, FF)
    for k in range(K):
        cuts = sorted(set(int(c) for c in rng.integers(1, 2 * FF, size=int(rng.integers(0, 4)))))
        b = [0] + cuts + [2 * FF]
        for r0, r1 in zip(b[:-1], b[1:]):
            tasks.append(mk(flh, T.STREAM_DOT_IDX, fmt=fgu, w=dgu_w.ptr + r0 * rbg, w_bytes=(r1 - r0) * rbg,
                            x=dxn.ptr, y=dgu.ptr + 4 * (k * 2 * FF + r0), rows=r1 - r0, cols=D,
                            aux=dids.ptr + 4 * k, aux2=egu))
    for k in range(K):
        hk = dh.ptr + 4 * k * stF
        tasks.append(mk(flh, T.SILU_MUL, aux=host(flh.SiluMulP(dgu.ptr + 4 * k * 2 * FF,
                                                               dgu.ptr + 4 * (k * 2 * FF + FF), hk, FF))))
        tasks.append(mk(flh, T.ACT_Q8, x=hk, y=hk + flh.xq_offset(FF), rows=FF // 32, cols=FF))
        tasks.append(mk(flh, T.STREAM_DOT_IDX, fmt=fdn, w=ddn_w.ptr, w_bytes=D * rbd, x=hk,
                        y=dparts.ptr + 4 * k * D, rows=D, cols=FF, aux=dids.ptr + 4 * k, aux2=edn))
    tasks.append(mk(flh, T.WMERGE, aux=host(flh.WmergeP(dparts.ptr, dgates.ptr, dx.ptr, None, dout.ptr, 1.0, K, D,
                                                        0))))
    tasks.append(mk(flh, T.SIGNAL))
    flh.exec_tasks(tasks, gpu, i8_mask=I8_ALL)

    # each stage on the device's own input
    xn = dxn.download(np.float32, stD, gpu)
    ref = orc.rmsnorm(x, wn, 1e-5)
    assert np.all(np.abs(xn[:D] - ref) <= D * 2.0 ** -24 * np.abs(ref) + 2 * np.spacing(np.abs(ref)))
    n8 = x_alloc_bytes(D) // 4
    assert np.array_equal(xn[:n8].view(np.uint8), orc.act_q8(xn[:D]).view(np.uint8)), "xn appendices"
    if shared:
        want = np.zeros(FF, np.float32)
        orc.stream_dot(Q4_K, ws, FF, D, xn, want, i8_mask=I8_ALL, threads=8)
        assert np.array_equal(bits(dsy.download(np.float32, FF, gpu)), bits(want)), "shared expert"
    ids, gates = orc.router_sel(logits, K, norm=norm)
    gids = dids.download(np.uint32, K, gpu)
    ggates = dgates.download(np.float32, K, gpu)
    assert np.array_equal(gids, ids)
    assert np.allclose(ggates, gates, rtol=2e-6, atol=1e-30)
    gu = dgu.download(np.float32, K * 2 * FF, gpu)
    h = dh.download(np.float32, K * stF, gpu)
    parts = dparts.download(np.float32, K * D, gpu)
    for k in range(K):
        want = np.zeros(2 * FF, np.float32)
        orc.stream_dot(fgu, wgu, 2 * FF, D, xn, want, id_slot=int(ids[k]), estride=egu, i8_mask=I8_ALL, threads=8)
        guk = gu[k * 2 * FF:(k + 1) * 2 * FF]
        assert np.array_equal(bits(guk), bits(want)), f"gate/up slot {k}"
        hk = h[k * stF:(k + 1) * stF]
        assert np.allclose(hk[:FF], orc.silu_mul(guk[:FF], guk[FF:]), rtol=4e-7, atol=1e-30)
        nf = x_alloc_bytes(FF) // 4
        assert np.array_equal(hk[:nf].view(np.uint8), orc.act_q8(hk[:FF]).view(np.uint8)), f"h appendices {k}"
        want = np.zeros(D, np.float32)
        orc.stream_dot(fdn, wdn, D, FF, hk, want, id_slot=int(ids[k]), estride=edn, i8_mask=I8_ALL, threads=8)
        assert np.array_equal(bits(parts[k * D:(k + 1) * D]), bits(want)), f"down slot {k}"
    want = orc.wmerge(parts.reshape(K, D), ggates, x, None)
    assert np.array_equal(bits(dout.download(np.float32, D, gpu)), bits(want))
