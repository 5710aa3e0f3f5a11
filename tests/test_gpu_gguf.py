"""GGUF -> HBM on the GPU: flh_gguf_upload / flh_gguf_upload_all put every
payload byte on the device at the file's offsets (checked by download), and
STREAM_DOT / STREAM_DOT_IDX straight from the uploaded weights equal the
oracle run on the mapped file bytes, bit for bit.  The large case crosses the
pinned staging ring several times and reports the upload rate.
"""
import os
import time

import numpy as np
import pytest

from oracle import col_stride_floats
from gguf_writer import GgufFile
import gguf_writer as gw
from util import sane_rows, activations
from test_gpu_parity import bits, say, dev_cols

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = os.path.join(HERE, "golden", "gguf")
GGML = {1: gw.GGML_Q8_0, 2: gw.GGML_Q5_0, 3: gw.GGML_Q4_K, 4: gw.GGML_Q6_K}


def download(flh, gpu, addr, n):
    out = np.empty(n, dtype=np.uint8)
    flh.check(flh.lib().flh_download(out.ctypes.data, addr, n, gpu.handle))
    return out


@pytest.mark.parametrize("name", ["basic.gguf", "kv_types.gguf", "model-00001-of-00003.gguf"])
def test_upload_all_bytes(flh, gpu, name):
    say("gguf upload_all", name)
    arena = flh.Arena(64 << 20)
    try:
        with flh.Gguf(os.path.join(FIX, name)) as g:
            ptrs = g.upload_all(arena, gpu)
            for t, p in zip(g.tensors(), ptrs):
                if t.nbytes == 0:
                    assert p is None
                    continue
                assert p % 32 == 0 or g.alignment() != 32
                assert np.array_equal(download(flh, gpu, p, t.nbytes), g.data(t)), t.name
    finally:
        arena.close()


def test_upload_one_tensor(flh, gpu):
    say("gguf upload one")
    with flh.Gguf(os.path.join(FIX, "kv_types.gguf")) as g:
        t = g.find("q6.wide")
        buf = flh.DeviceBuffer(t.nbytes + 64)
        g.upload(t, buf, gpu)
        assert np.array_equal(buf.download(np.uint8, t.nbytes, gpu), g.data(t))
        with pytest.raises(flh.FlhError):
            g.upload(t, buf, gpu, dst_bytes=t.nbytes - 1)
        with pytest.raises(flh.FlhError):
            g.upload(g.find("q4_0.unsized"), buf, gpu)


def test_dots_from_uploaded_weights(flh, orc, gpu, tmp_path):
    """Weights written to a GGUF, read back and uploaded, then STREAM_DOT at
    decode shapes (and an expert stack through STREAM_DOT_IDX): device output
    equals the oracle on the mapped bytes."""
    rng = np.random.default_rng(4242)
    f = GgufFile(3)
    specs = [("blk.0.attn_q.weight", 3, 4096, 512), ("output.weight", 4, 4096, 300),
             ("blk.0.ffn_down.weight", 1, 1408, 96), ("blk.0.attn_v.weight", 2, 2048, 64)]
    for name, fmt, cols, rows in specs:
        f.add_tensor(name, GGML[fmt], (cols, rows), sane_rows(fmt, rows, cols, rng))
    ne = 4
    f.add_tensor("blk.1.ffn_up_exps.weight", gw.GGML_Q4_K, (2048, 40, ne),
                 sane_rows(3, 40 * ne, 2048, rng))
    path = str(tmp_path / "m.gguf")
    f.write(path)
    arena = flh.Arena(256 << 20)
    try:
        with flh.Gguf(path) as g:
            ptrs = g.upload_all(arena, gpu)
            for name, fmt, cols, rows in specs:
                say("gguf dot", name)
                w = g.weight(name)
                assert (w.fmt, w.rows, w.cols) == (fmt, rows, cols)
                xs = activations(2, cols, rng)
                st = col_stride_floats(cols)
                dx, _ = dev_cols(flh, gpu, xs, st)
                flh.act_q8(dx, cols, gpu, nx=2, xstride=st)
                ref_x = orc.act_q8_cols(xs, st)
                dy = flh.DeviceBuffer(2 * rows * 4)
                dy.zero(gpu)
                flh.stream_dot(fmt, ptrs[w.tensor], rows, cols, dx, dy, gpu, nx=2, xstride=st,
                               ystride=rows, w_bytes=w.w_bytes)
                want = np.zeros(2 * rows, dtype=np.float32)
                orc.stream_dot(fmt, g.data(g.find(name)), rows, cols, ref_x, want, nx=2,
                               xstride=st, ystride=rows)
                got = dy.download(np.float32, 2 * rows, gpu)
                assert np.array_equal(bits(got), bits(want)), name
            say("gguf idx dot")
            w = g.weight("blk.1.ffn_up_exps.weight")
            assert w.nexp == ne and w.estride == w.w_bytes
            xs = activations(1, w.cols, rng)
            st = col_stride_floats(w.cols)
            dx, _ = dev_cols(flh, gpu, xs, st)
            flh.act_q8(dx, w.cols, gpu)
            ref_x = orc.act_q8_cols(xs, st)
            host = g.data(g.find("blk.1.ffn_up_exps.weight"))
            for e in range(ne):
                slot = flh.DeviceBuffer.from_array(np.array([e], dtype=np.uint32), gpu)
                dy = flh.DeviceBuffer(w.rows * 4)
                dy.zero(gpu)
                flh.stream_dot(w.fmt, ptrs[w.tensor], w.rows, w.cols, dx, dy, gpu, id_slot=slot,
                               estride=w.estride, w_bytes=w.w_bytes)
                want = np.zeros(w.rows, dtype=np.float32)
                orc.stream_dot(w.fmt, host, w.rows, w.cols, ref_x, want, id_slot=e,
                               estride=w.estride)
                assert np.array_equal(bits(dy.download(np.float32, w.rows, gpu)), bits(want)), e
    finally:
        arena.close()


def test_large_upload_through_staging_ring(flh, gpu, tmp_path):
    """A 1.1 GiB file (many passes over the 4 x 64 MiB pinned ring, two
    shards): every byte lands at its offset; prints the host->HBM rate."""
    rng = np.random.default_rng(77)
    nb = 600 << 20
    paths = []
    for s in (1, 2):
        f = GgufFile(3)
        f.add_kv("split.count", gw.U16, 2)
        payload = rng.integers(0, 256, size=nb // 8, dtype=np.uint64).view(np.uint8)
        f.add_tensor(f"big{s}", gw.GGML_Q8_0, (32, nb // 34), payload[:(nb // 34) * 34])
        f.add_tensor(f"tail{s}", gw.GGML_F32, (1000,), rng.standard_normal(1000).astype(np.float32))
        p = str(tmp_path / f"big-0000{s}-of-00002.gguf")
        f.write(p)
        paths.append(p)
        del payload, f
    arena = flh.Arena(nb * 2 + (64 << 20))
    try:
        with flh.Gguf(paths[0]) as g:
            total = sum(t.nbytes for t in g.tensors())
            gpu.sync()
            t0 = time.perf_counter()
            ptrs = g.upload_all(arena, gpu)
            dt = time.perf_counter() - t0
            say(f"gguf upload_all {total / 2**30:.2f} GiB in {dt * 1e3:.1f} ms = "
                f"{total / dt / 1e9:.1f} GB/s (page cache -> HBM)")
            for t, p in zip(g.tensors(), ptrs):
                assert np.array_equal(download(flh, gpu, p, t.nbytes), g.data(t)), t.name
    finally:
        arena.close()
