"""Every tuning switch read at flh_init changes launch shapes only.

Each case sets one switch to a non-default value and runs a shape whose path
that switch steers (fused ACT_Q8 width, the streaming kernel's grid / ring,
the register kernel's grid / ring, the matrix-core prologue and column
threshold, the upload's copy threads).  The result must equal the default
run's bits and the oracle's (fl_dot_i8k_q4_K / fl_dot_i8k_q6_K,
src/runtime/quants.h:538-594).
"""
import numpy as np
import pytest

from oracle import Q4_K, Q6_K, col_stride_floats
from util import tuned, sane_rows, activations
from test_gpu_parity import bits, say, dev_cols

pytestmark = pytest.mark.gpu


def run(flh, orc, gpu, fmt, w, rows, cols, xs, misalign, fused):
    """y = 0 += W x for nx columns; the weights start `misalign` bytes into
    their buffer (4: only the register kernel takes them)."""
    nx = xs.shape[0]
    st = col_stride_floats(cols)
    dx, _ = dev_cols(flh, gpu, xs, st)
    if fused:
        assert nx == 1
        dy = flh.DeviceBuffer.from_array(np.zeros(rows, np.float32), gpu)
        dw = flh.DeviceBuffer.from_array(w, gpu)
        flh.act_q8_stream_dot(fmt, dw, rows, cols, dx, dy, gpu)
    else:
        flh.act_q8(dx, cols, gpu, nx=nx, xstride=st)
        dy = flh.DeviceBuffer.from_array(np.zeros(nx * rows, np.float32), gpu)
        dw = flh.DeviceBuffer.from_array(np.concatenate([np.zeros(misalign, np.uint8), w]), gpu)
        flh.stream_dot(fmt, dw.ptr + misalign, rows, cols, dx, dy, gpu, nx=nx, xstride=st, ystride=rows)
    got = dy.download(np.float32, nx * rows, gpu)
    want = np.zeros(nx * rows, np.float32)
    orc.stream_dot(fmt, w, rows, cols, orc.act_q8_cols(xs, st), want, nx=nx, xstride=st, ystride=rows, threads=8)
    return got, want


# (switch, value, format, rows, cols, columns, weight misalignment, fused ACT_Q8)
CASES = [
    ("FLH_FUSE_MAX_COLS", "16384", Q4_K, 300, 14336, 1, 0, True),    # fused at 14336 columns
    ("FLH_FUSE_MAX_COLS", "0", Q4_K, 300, 4096, 1, 0, True),         # never fused
    ("FLH_KS_TUNE", "1,0,3,2", Q6_K, 1000, 14336, 1, 0, False),      # streaming kernel: 3-deep ring
    ("FLH_KS_TUNE", "2,16,2,1", Q6_K, 1000, 4096, 2, 0, False),
    ("FLH_KQ_TUNE", "2,8,4", Q4_K, 257, 4096, 1, 4, False),          # register kernel
    ("FLH_KQ_TUNE", "1,0,1", Q6_K, 257, 2048, 2, 4, False),
    ("FLH_MFMA_PRO", "1", Q4_K, 1000, 4096, 4, 0, False),            # matrix cores: 1-chunk prologue
    ("FLH_MFMA_MIN_COLS", "2", Q4_K, 1000, 4096, 2, 0, False),       # matrix cores at 2 columns
    ("FLH_MFMA_OWN", "0", Q4_K, 14336, 4096, 8, 0, False),          # matrix cores: parked terms + fold
    ("FLH_MFMA_OWN", "0", Q4_K, 1000, 4096, 3, 0, False),
    ("FLH_MFMA_OWN", "0", Q4_K, 777, 2816, 16, 0, False),
    ("FLH_MFMA_OWN", "0", Q4_K, 4096, 14336, 4, 0, False),          # one tile per batch: split chains
    ("FLH_MFMA_OWN", "0", Q4_K, 4096, 14336, 2, 0, False),
    ("FLH_MFMA_OWN", "0", Q4_K, 3000, 4096, 8, 0, False),
]


@pytest.mark.parametrize("ntok", [3, 8])
def test_moe_register_sums_keep_bits(flh, gpu, ntok):
    """The grouped matrix-core expert dots with register accumulators (the
    default) and with parked terms and a fold pass (FLH_MFMA_OWN=0) give the
    same bits for every (token, slot) pair."""
    say("tuning moe own", ntok)
    E, K, rows, cols = 6, 2, 1500, 4096
    rng = np.random.default_rng(ntok)
    from oracle import row_bytes
    rb = rows * row_bytes(Q4_K, cols)
    w = sane_rows(Q4_K, E * rows, cols, rng)
    xs = activations(ntok, cols, rng, outliers=True)
    st = col_stride_floats(cols)
    ids = np.array([rng.permutation(E)[:K] for _ in range(ntok)], dtype=np.uint32).reshape(-1)
    dx, _ = dev_cols(flh, gpu, xs, st)
    flh.act_q8(dx, cols, gpu, nx=ntok, xstride=st)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    did = flh.DeviceBuffer.from_array(ids, gpu)
    out = []
    for env in ({}, {"FLH_MFMA_OWN": "0"}):
        dy = flh.DeviceBuffer(ntok * K * rows * 4)
        dy.zero(gpu)
        with tuned(flh, **env):
            flh.moe_dot(Q4_K, dw, rb, rows, cols, did, ntok, K, E, dx, st, False, dy, rows, gpu)
        out.append(dy.download(np.float32, ntok * K * rows, gpu))
    assert np.array_equal(bits(out[0]), bits(out[1]))


@pytest.mark.parametrize("name,value,fmt,rows,cols,nx,mis,fused", CASES)
def test_switch_keeps_bits(flh, orc, gpu, name, value, fmt, rows, cols, nx, mis, fused):
    say("tuning", name, value, fmt, rows, cols, nx, mis, fused)
    rng = np.random.default_rng(rows + cols + nx)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    base, want = run(flh, orc, gpu, fmt, w, rows, cols, xs, mis, fused)
    assert np.array_equal(bits(base), bits(want))
    with tuned(flh, **{name: value}):
        got, _ = run(flh, orc, gpu, fmt, w, rows, cols, xs, mis, fused)
    assert np.array_equal(bits(got), bits(want))


def test_gguf_copy_threads_keep_bytes(flh, gpu, tmp_path):
    """FLH_GGUF_THREADS=1 and =3: a tensor above the parallel-copy threshold
    (4 MiB) lands byte for byte either way."""
    import gguf_writer as gw
    rng = np.random.default_rng(5)
    payload = rng.integers(0, 256, size=(8 << 20) // 34 * 34, dtype=np.uint8)
    f = gw.GgufFile(3)
    f.add_tensor("w", gw.GGML_Q8_0, (32, payload.size // 34), payload)
    p = str(tmp_path / "w.gguf")
    f.write(p)
    for n in ("1", "3"):
        say("gguf threads", n)
        with tuned(flh, FLH_GGUF_THREADS=n):
            with flh.Gguf(p) as g:
                t = g.find("w")
                buf = flh.DeviceBuffer(t.nbytes + 64)
                g.upload(t, buf, gpu)
                assert np.array_equal(buf.download(np.uint8, t.nbytes, gpu), payload)
