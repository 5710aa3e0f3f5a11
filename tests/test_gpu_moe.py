"""MoE decode path on the GPU: grouped expert matvec, router, silu*up, merge.

The grouped kernel must reproduce, bit for bit, the per-(token, slot)
STREAM_DOT_IDX tiles the reference emits (src/model/decoder.cpp:941-996),
checked against the oracle.  The decode ops that call expf (router softmax,
silu) use the device libm, so they are compared within float tolerance; the
whole FFN layer is held to the north-star bar (1e-3 of max |y|).
"""
import numpy as np
import pytest

from oracle import Q4_K, Q6_K, col_stride_floats, row_bytes
from util import sane_rows, activations

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def say(*a):
    print("[case]", *a, flush=True)


def route(orc, ntok, E, K, rng):
    logits = rng.standard_normal((ntok, E)).astype(np.float32)
    ids = np.zeros((ntok, K), dtype=np.uint32)
    gates = np.zeros((ntok, K), dtype=np.float32)
    for t in range(ntok):
        ids[t], gates[t] = orc.router_sel(logits[t], K, norm=1)
    return logits, ids, gates


@pytest.mark.parametrize("fmt", [Q4_K, Q6_K])
@pytest.mark.parametrize("ntok,rows,cols,per_slot", [(1, 300, 1024, False), (3, 64, 2816, False),
                                                     (8, 257, 4096, False), (8, 96, 2048, True),
                                                     (5, 40, 14336, True), (16, 1024, 4096, False),
                                                     (8, 4096, 14336, True)])
def test_grouped_expert_dot_bitwise(flh, orc, gpu, fmt, ntok, rows, cols, per_slot):
    grouped_dot_case(flh, orc, gpu, fmt, ntok, rows, cols, per_slot)


def test_grouped_expert_dot_mixtral_gate_up_batch8(flh, orc, gpu):
    """The benchmark's MoE shape: 8 experts of 28672x4096 Q4_K (fused gate/up),
    8 tokens routed top-2 (matrix-core grouped kernel), bitwise."""
    grouped_dot_case(flh, orc, gpu, Q4_K, 8, 28672, 4096, False)


@pytest.mark.parametrize("rows,cols,per_slot", [(28672, 4096, False), (4096, 14336, True)])
def test_grouped_expert_dot_mixtral_batch1(flh, orc, gpu, rows, cols, per_slot):
    """The benchmark's MoE batch-1 shapes (one token, top-2 of 8 experts):
    the fused gate/up 28672x4096 and the down 4096x14336 per expert on the
    grouped streaming kernel, bitwise."""
    grouped_dot_case(flh, orc, gpu, Q4_K, 1, rows, cols, per_slot)


def grouped_dot_case(flh, orc, gpu, fmt, ntok, rows, cols, per_slot):
    say("moe_dot", fmt, ntok, rows, cols, per_slot)
    rng = np.random.default_rng(ntok * 31 + rows + cols + fmt)
    E, K = 8, 2
    _, ids, _ = route(orc, ntok, E, K, rng)
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
    di = flh.DeviceBuffer.from_array(ids.ravel(), gpu)
    flh.moe_dot(fmt, dw, estride, rows, cols, di, ntok, K, E, dx, st, per_slot, dy, rows, gpu)
    got = dy.download(np.float32, y0.size, gpu)
    want = y0.copy()
    for t in range(ntok):
        for k in range(K):
            i = t * K + k
            xi = i if per_slot else t
            yi = want[i * rows:(i + 1) * rows]
            orc.stream_dot(fmt, w, rows, cols, ref_x[xi * st:(xi + 1) * st], yi,
                           id_slot=int(ids[t, k]), estride=estride, threads=8)
            want[i * rows:(i + 1) * rows] = yi
    assert np.array_equal(bits(got), bits(want))


def test_router_matches_reference_order(flh, orc, gpu, golden):
    """Top-k ids equal the reference's (ties -> lower id); gates to float tolerance."""
    say("router")
    for name, K, norm in (("router_kat_in", 3, 0), ("router_kat_in", 3, 1)):
        lg = golden[name]
        d_l = flh.DeviceBuffer.from_array(lg, gpu)
        d_i = flh.DeviceBuffer(4 * K)
        d_g = flh.DeviceBuffer(4 * K)
        flh.router_sel(d_l, 1, lg.size, K, norm, 1.0, d_i, d_g, gpu)
        ids = d_i.download(np.uint32, K, gpu)
        g = d_g.download(np.float32, K, gpu)
        assert list(ids) == list(golden[f"router_kat_ids_{norm}"])
        assert np.allclose(g, golden[f"router_kat_gates_{norm}"], rtol=2e-6, atol=0)
    lg = golden["router_in"]
    d_l = flh.DeviceBuffer.from_array(lg, gpu)
    d_i = flh.DeviceBuffer(4 * 2 * lg.shape[0])
    d_g = flh.DeviceBuffer(4 * 2 * lg.shape[0])
    flh.router_sel(d_l, lg.shape[0], 8, 2, 1, 1.0, d_i, d_g, gpu)
    assert np.array_equal(d_i.download(np.uint32, 2 * lg.shape[0], gpu).reshape(-1, 2), golden["router_ids"])
    assert np.allclose(d_g.download(np.float32, 2 * lg.shape[0], gpu).reshape(-1, 2),
                       golden["router_gates"], rtol=2e-6, atol=0)


def test_silu_mul_and_wmerge(flh, gpu, golden):
    say("silu/wmerge")
    g, u = golden["silu_g"], golden["silu_u"]
    dg, du = flh.DeviceBuffer.from_array(g, gpu), flh.DeviceBuffer.from_array(u, gpu)
    dh = flh.DeviceBuffer(g.nbytes)
    flh.silu_mul(dg, du, dh, g.size, 1, 0, 0, gpu)
    h = dh.download(np.float32, g.size, gpu)
    assert np.allclose(h, golden["silu_h"], rtol=4e-7, atol=1e-30)
    parts, gates, add1 = golden["wm_parts"], golden["wm_gates"], golden["wm_add1"]
    dp = flh.DeviceBuffer.from_array(parts, gpu)
    dgt = flh.DeviceBuffer.from_array(gates, gpu)
    da = flh.DeviceBuffer.from_array(add1, gpu)
    dy = flh.DeviceBuffer(add1.nbytes)
    flh.wmerge(dp, dgt, da, None, dy, 1.0, 2, add1.size, 0, 1, 0, 0, gpu)
    assert np.array_equal(bits(dy.download(np.float32, add1.size, gpu)), bits(golden["wm_y"]))


@pytest.mark.parametrize("ntok", [1, 8])
def test_moe_ffn_layer_end_to_end(flh, orc, gpu, ntok):
    """router -> grouped gate/up -> silu*up -> ACT_Q8 -> grouped down ->
    weighted merge + residual, against the oracle's per-token reference
    sequence (decoder.cpp:941-1040), within 1e-3 of max |y|."""
    say("moe ffn", ntok)
    rng = np.random.default_rng(ntok)
    E, K, D, F = 8, 2, 1024, 2048
    logits, ids_ref, gates_ref = route(orc, ntok, E, K, rng)
    wgu = flh.quantize_host(Q4_K, (rng.standard_normal((E * 2 * F, D)) * 0.02).astype(np.float32))
    wdn = flh.quantize_host(Q4_K, (rng.standard_normal((E * D, F)) * 0.02).astype(np.float32))
    gu_stride, dn_stride = 2 * F * row_bytes(Q4_K, D), D * row_bytes(Q4_K, F)
    xs = activations(ntok, D, rng)
    resid = rng.standard_normal((ntok, D)).astype(np.float32)
    stD, stF = col_stride_floats(D), col_stride_floats(F)
    # ---- device
    xb = np.zeros(ntok * stD, dtype=np.float32)
    for t in range(ntok):
        xb[t * stD:t * stD + D] = xs[t]
    dx = flh.DeviceBuffer.from_array(xb, gpu)
    dlg = flh.DeviceBuffer.from_array(logits, gpu)
    dids, dgat = flh.DeviceBuffer(4 * ntok * K), flh.DeviceBuffer(4 * ntok * K)
    dgu_w, ddn_w = flh.DeviceBuffer.from_array(wgu, gpu), flh.DeviceBuffer.from_array(wdn, gpu)
    ygu = flh.DeviceBuffer(4 * ntok * K * 2 * F)
    ygu.zero(gpu)
    h = flh.DeviceBuffer(4 * ntok * K * stF)
    h.zero(gpu)
    ydn = flh.DeviceBuffer(4 * ntok * K * D)
    ydn.zero(gpu)
    dres = flh.DeviceBuffer.from_array(resid, gpu)
    yo = flh.DeviceBuffer(4 * ntok * D)
    flh.act_q8(dx, D, gpu, nx=ntok, xstride=stD)
    flh.router_sel(dlg, ntok, E, K, 1, 1.0, dids, dgat, gpu)
    flh.moe_dot(Q4_K, dgu_w, gu_stride, 2 * F, D, dids, ntok, K, E, dx, stD, False, ygu, 2 * F, gpu)
    flh.silu_mul(ygu, ygu.ptr + 4 * F, h, F, ntok * K, 2 * F, stF, gpu)
    flh.act_q8(h, F, gpu, nx=ntok * K, xstride=stF)
    flh.moe_dot(Q4_K, ddn_w, dn_stride, D, F, dids, ntok, K, E, h, stF, True, ydn, D, gpu)
    flh.wmerge(ydn, dgat, dres, None, yo, 1.0, K, D, 0, ntok, K * D, D, gpu)
    got = yo.download(np.float32, ntok * D, gpu).reshape(ntok, D)
    assert np.array_equal(dids.download(np.uint32, ntok * K, gpu).reshape(ntok, K), ids_ref)
    # ---- oracle, per token and slot as the reference graph runs it
    want = np.zeros((ntok, D), dtype=np.float32)
    for t in range(ntok):
        xq = orc.act_q8_cols(xs[t:t + 1], stD)
        parts = np.zeros((K, D), dtype=np.float32)
        for k in range(K):
            e = int(ids_ref[t, k])
            yg = np.zeros(2 * F, dtype=np.float32)
            orc.stream_dot(Q4_K, wgu, 2 * F, D, xq, yg, id_slot=e, estride=gu_stride)
            hh = orc.silu_mul(yg[:F], yg[F:])
            hq = orc.act_q8_cols(hh[None, :], stF)
            yd = np.zeros(D, dtype=np.float32)
            orc.stream_dot(Q4_K, wdn, D, F, hq, yd, id_slot=e, estride=dn_stride)
            parts[k] = yd
        want[t] = orc.wmerge(parts, gates_ref[t], add1=resid[t])
    err = np.max(np.abs(got - want))
    assert err <= 1e-3 * np.max(np.abs(want)), err


@pytest.mark.parametrize("n,ncol", [(14336, 3), (1000, 2), (256, 1)])
def test_silu_mul_act_q8_fused_equals_separate(flh, gpu, n, ncol):
    """The fused SILU_MUL+ACT_Q8 launch writes the bytes of SILU_MUL followed
    by ACT_Q8 (h and both appendices of every column)."""
    say("silu+act_q8", n, ncol)
    from oracle import col_stride_floats, x_alloc_bytes
    rng = np.random.default_rng(n + ncol)
    gs = 2 * n + 5
    gu = (rng.standard_normal(ncol * gs) * 3).astype(np.float32)
    st = col_stride_floats(n)
    dgu = flh.DeviceBuffer.from_array(gu, gpu)
    h1 = flh.DeviceBuffer.from_array(np.zeros(ncol * st, np.float32), gpu)
    h2 = flh.DeviceBuffer.from_array(np.zeros(ncol * st, np.float32), gpu)
    flh.silu_mul(dgu, dgu.ptr + 4 * n, h1, n, ncol, gs, st, gpu)
    flh.act_q8(h1, n, gpu, nx=ncol, xstride=st)
    flh.silu_mul_act_q8(dgu, dgu.ptr + 4 * n, h2, n, ncol, gs, st, gpu)
    a = h1.download(np.float32, ncol * st, gpu).view(np.uint8)
    b = h2.download(np.float32, ncol * st, gpu).view(np.uint8)
    for c in range(ncol):
        lo = c * st * 4
        assert np.array_equal(a[lo:lo + x_alloc_bytes(n)], b[lo:lo + x_alloc_bytes(n)]), f"column {c}"


@pytest.mark.parametrize("E,K,norm", [(8, 2, 1), (64, 6, 0), (16, 4, 1), (100, 8, 1)])
def test_router_ties_and_widths(flh, orc, gpu, E, K, norm):
    """Equal weights resolve to the lower expert id (strict > in expert order,
    decode_params.h:234-265); one-wave router (E <= 64) and per-thread router
    (E > 64) both."""
    say("router ties", E, K, norm)
    rng = np.random.default_rng(E * 7 + K)
    ntok = 5
    lg = rng.integers(-3, 4, size=(ntok, E)).astype(np.float32) * 0.5   # many exact ties
    d_l = flh.DeviceBuffer.from_array(lg.ravel(), gpu)
    d_i = flh.DeviceBuffer(ntok * K * 4)
    d_g = flh.DeviceBuffer(ntok * K * 4)
    flh.router_sel(d_l, ntok, E, K, norm, 1.0, d_i, d_g, gpu)
    ids = d_i.download(np.uint32, ntok * K, gpu).reshape(ntok, K)
    g = d_g.download(np.float32, ntok * K, gpu).reshape(ntok, K)
    for t in range(ntok):
        wi, wg = orc.router_sel(lg[t], K, norm=norm)
        assert list(ids[t]) == list(wi)
        assert np.allclose(g[t], wg, rtol=2e-6, atol=0)


@pytest.mark.parametrize("fmt,ntok,rows,cols,per_slot,norm,E,K", [
    (Q4_K, 1, 1024, 4096, False, 1, 8, 2), (Q4_K, 8, 512, 4096, False, 1, 8, 2),
    (Q4_K, 8, 256, 14336, True, 0, 8, 2), (Q6_K, 3, 300, 2048, False, 1, 8, 2),
    (Q4_K, 5, 128, 1024, False, 1, 64, 8), (Q6_K, 32, 64, 512, True, 1, 16, 8),
])
def test_router_moe_dot_fused_equals_separate(flh, gpu, fmt, ntok, rows, cols, per_slot, norm, E, K):
    """flh_router_moe_dot (routing inside the grouped kernels) writes the ids,
    gates and y of flh_router_sel followed by flh_moe_dot, bit for bit, incl.
    tied logits (lowest id wins), 64 experts and top-8."""
    say("router+moe", fmt, ntok, rows, cols, per_slot, norm, E, K)
    rng = np.random.default_rng(ntok * 7 + rows + cols + E)
    logits = rng.standard_normal((ntok, E)).astype(np.float32)
    logits[0, 1] = logits[0, 3] = np.max(logits[0]) + 0.5            # a tie for the top weight
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
    dw = flh.DeviceBuffer.from_array(w, gpu)
    dl = flh.DeviceBuffer.from_array(logits, gpu)
    y0 = rng.standard_normal(ntok * K * rows).astype(np.float32)
    outs = []
    for fused in (False, True):
        di, dg = flh.DeviceBuffer(4 * ntok * K), flh.DeviceBuffer(4 * ntok * K)
        dy = flh.DeviceBuffer.from_array(y0, gpu)
        if fused:
            flh.router_moe_dot(fmt, dw, estride, rows, cols, dl, ntok, E, K, norm, 0.75, di, dg, dx, st,
                               per_slot, dy, rows, gpu)
        else:
            flh.router_sel(dl, ntok, E, K, norm, 0.75, di, dg, gpu)
            flh.moe_dot(fmt, dw, estride, rows, cols, di, ntok, K, E, dx, st, per_slot, dy, rows, gpu)
        outs.append((di.download(np.uint32, ntok * K, gpu), bits(dg.download(np.float32, ntok * K, gpu)),
                     bits(dy.download(np.float32, y0.size, gpu))))
    assert list(outs[0][0][:2]) == [1, 3]                               # tie -> lower id first
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("ntok,rows,cols,per_slot", [(8, 300, 4096, False), (6, 130, 2816, True)])
def test_grouped_expert_dot_k_halves_bitwise(flh, orc, gpu, ntok, rows, cols, per_slot):
    """The grouped matrix-core kernel with K halves forced (the mode wide
    expert inputs take when the whole activations do not fit LDS), bitwise."""
    from util import tuned
    with tuned(flh, FLH_MFMA_TUNE="2,0,1"):
        grouped_dot_case(flh, orc, gpu, Q4_K, ntok, rows, cols, per_slot)


@pytest.mark.parametrize("cfg", ["1", "1,8,1,0", "1,4,2,0,255"])
@pytest.mark.parametrize("rows,cols,per_slot,E,K", [(300, 1024, False, 8, 2), (97, 14336, True, 8, 2),
                                                    (1001, 4096, False, 64, 8), (64, 2048, True, 16, 4)])
def test_moe_one_token_superblock_kernel(flh, orc, gpu, cfg, rows, cols, per_slot, E, K):
    """One token (the superblock-per-lane routed launch, one workgroup row per
    pair): bitwise against the oracle and against the grouped streaming kernel
    (FLH_SBL=0); a pair whose id is out of range leaves its y untouched."""
    from util import tuned
    say("moe one token", cfg, rows, cols, per_slot, E, K)
    rng = np.random.default_rng(rows + cols + E * K)
    ids = rng.choice(E, size=K, replace=False).astype(np.uint32)
    ids[K - 1] = E + 3                                   # not routed
    rb = row_bytes(Q4_K, cols)
    estride = rows * rb
    w = sane_rows(Q4_K, rows * E, cols, rng)
    nx = K if per_slot else 1
    xs = activations(nx, cols, rng, outliers=True)
    st = col_stride_floats(cols)
    buf = np.zeros(nx * st, dtype=np.float32)
    for p in range(nx):
        buf[p * st:p * st + cols] = xs[p]
    dx = flh.DeviceBuffer.from_array(buf, gpu)
    flh.act_q8(dx, cols, gpu, nx=nx, xstride=st)
    ref_x = orc.act_q8_cols(xs, st)
    y0 = rng.standard_normal(K * rows).astype(np.float32)
    want = y0.copy()
    for k in range(K - 1):
        xi = k if per_slot else 0
        yk = want[k * rows:(k + 1) * rows]
        orc.stream_dot(Q4_K, w, rows, cols, ref_x[xi * st:(xi + 1) * st], yk, id_slot=int(ids[k]),
                       estride=estride, threads=8)
        want[k * rows:(k + 1) * rows] = yk
    dw = flh.DeviceBuffer.from_array(w, gpu)
    di = flh.DeviceBuffer.from_array(ids, gpu)
    outs = []
    for c in (cfg, "0"):
        with tuned(flh, FLH_SBL=c):
            dy = flh.DeviceBuffer.from_array(y0, gpu)
            flh.moe_dot(Q4_K, dw, estride, rows, cols, di, 1, K, E, dx, st, per_slot, dy, rows, gpu)
            outs.append(dy.download(np.float32, y0.size, gpu))
    assert np.array_equal(bits(outs[0]), bits(want))
    assert np.array_equal(bits(outs[1]), bits(want))


Q8_0, Q5_0, IQ2_XXS, IQ3_XXS = 1, 2, 5, 6


@pytest.mark.parametrize("cols", [2048, 14336])
@pytest.mark.parametrize("fmt", [Q8_0, Q5_0, IQ2_XXS, IQ3_XXS])
@pytest.mark.parametrize("ntok,per_slot,fused", [(1, False, False), (3, True, False), (5, False, True),
                                                 (2, True, True)])
def test_moe_block32_formats(flh, orc, gpu, fmt, ntok, per_slot, fused, cols):
    """Expert dots of the 32-weight-block formats (one workgroup row per
    routed pair): every pair's y equals the oracle's STREAM_DOT_IDX tile on
    the q8_1 int8 path, bit for bit, with the routing given as ids or fused
    (ids then equal the reference router's; gates within the expf tolerance).
    14336 columns: a down projection, two four-block halves per lane."""
    say("moe block32", fmt, ntok, per_slot, fused, cols)
    rng = np.random.default_rng(fmt * 11 + ntok * 3 + fused + cols)
    E, K, rows = 8, 2, 200 if cols == 2048 else 72
    logits, ids, gates = route(orc, ntok, E, K, rng)
    estride = rows * row_bytes(fmt, cols)
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
        assert np.allclose(dg.download(np.float32, ntok * K, gpu), gates.ravel(), rtol=2e-6, atol=0)   # expf
    else:
        di = flh.DeviceBuffer.from_array(ids.ravel(), gpu)
        flh.moe_dot(fmt, dw, estride, rows, cols, di, ntok, K, E, dx, st, per_slot, dy, rows, gpu)
    got = dy.download(np.float32, y0.size, gpu)
    want = y0.copy()
    i8 = 0b11110 | (1 << IQ2_XXS) | (1 << IQ3_XXS)
    for t in range(ntok):
        for k in range(K):
            i = t * K + k
            xi = i if per_slot else t
            yi = want[i * rows:(i + 1) * rows]
            orc.stream_dot(fmt, w, rows, cols, ref_x[xi * st:(xi + 1) * st], yi, id_slot=int(ids[t, k]),
                           estride=estride, i8_mask=i8, threads=8)
            want[i * rows:(i + 1) * rows] = yi
    assert np.array_equal(bits(got), bits(want))
