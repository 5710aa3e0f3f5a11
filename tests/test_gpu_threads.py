"""Two host threads issuing work on their own streams at once.

The C ABI is called concurrently (ctypes releases the interpreter lock for
each call): every thread runs a list of seeded dots (several formats,
columns and kernels, plus task tables) on its own stream and checks each
result against the oracle's, computed beforehand.  The library's host state
(the published tuning, the LDS-limit and static-LDS caches, the per-thread
error message) must not mix the threads' launches up: every output bit
equals the oracle's (the reference runs one stream per Runtime,
src/runtime/gpu_exec.cu:384-391; several Runtimes may run side by side).
"""
import threading

import numpy as np
import pytest

from oracle import Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, col_stride_floats
from util import sane_rows, activations
from test_gpu_parity import bits, dev_cols

pytestmark = pytest.mark.gpu

CASES = [(Q4_K, 3000, 4096, 1), (Q4_K, 1500, 4096, 4), (Q6_K, 2000, 2816, 1), (Q8_0, 700, 4096, 2),
         (Q5_0, 900, 2048, 1), (IQ2_XXS, 600, 4096, 1), (Q4_K, 800, 14336, 8), (Q6_K, 300, 4096, 3)]
I8_ALL = 0b1111110


def prepare(orc, case, seed):
    fmt, rows, cols, nx = case
    rng = np.random.default_rng(seed)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(nx, cols, rng, outliers=True)
    st = col_stride_floats(cols)
    y0 = rng.standard_normal(nx * rows).astype(np.float32)
    want = y0.copy()
    orc.stream_dot(fmt, w, rows, cols, orc.act_q8_cols(xs, st), want, nx=nx, xstride=st, ystride=rows,
                   i8_mask=I8_ALL, threads=8)
    return dict(fmt=fmt, rows=rows, cols=cols, nx=nx, w=w, xs=xs, st=st, y0=y0, want=want)


def test_two_threads_two_streams(flh, orc, gpu):
    jobs = [[prepare(orc, c, 10 * t + i) for i, c in enumerate(CASES[t::2] * 3)] for t in range(2)]
    print("[case] threads", [len(j) for j in jobs], flush=True)
    errors = []

    def run(t):
        try:
            s = flh.Stream()
            for j in jobs[t]:
                dx, _ = dev_cols(flh, s, j["xs"], j["st"])
                dw = flh.DeviceBuffer.from_array(j["w"], s)
                dy = flh.DeviceBuffer.from_array(j["y0"], s)
                flh.act_q8(dx, j["cols"], s, nx=j["nx"], xstride=j["st"])
                flh.stream_dot(j["fmt"], dw, j["rows"], j["cols"], dx, dy, s, nx=j["nx"], xstride=j["st"],
                               ystride=j["rows"], i8_mask=I8_ALL)
                got = dy.download(np.float32, j["y0"].size, s)
                if not np.array_equal(bits(got), bits(j["want"])):
                    errors.append((t, j["fmt"], j["rows"], j["cols"], j["nx"]))
                for b in (dx, dw, dy):
                    b.close()
            s.sync()
        except Exception as e:                  # reported by the main thread
            errors.append((t, repr(e)))

    th = [threading.Thread(target=run, args=(t,)) for t in range(2)]
    for x in th:
        x.start()
    for x in th:
        x.join(timeout=100)
    assert not any(x.is_alive() for x in th), "a thread did not finish"
    assert not errors, errors
