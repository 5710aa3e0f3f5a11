"""GPU parity at the BASELINE widths against the reference's own outputs.

Fixture: tests/golden/golden_wide.npz (tests/golden/make_wide_golden.py ran
the reference's exec_task_cpu on these seeded inputs; the inputs are
regenerated here and checked against the stored digests first).  Covers
Q4_K at 4096 and 14336 columns with 1, 2, 4 and 8 activation columns (the
streaming and matrix-core kernels), Q6_K at both widths, Q8_0 at 4096, and
the device Q8_0 weight quantizer against the reference's q8_1 block bytes.
Every comparison is bitwise.
"""
import os

import numpy as np
import pytest

from oracle import col_stride_floats
from wide_cases import WIDE_CASES, Q8_0_QUANT, wide_case_inputs, digest
from test_gpu_parity import bits, say, dev_cols

pytestmark = pytest.mark.gpu

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_wide.npz"))


@pytest.mark.parametrize("i", range(len(WIDE_CASES)))
def test_wide_dot_equals_reference(flh, gpu, i):
    fmt, rows, cols, nx, seed = WIDE_CASES[i]
    say("wide golden", fmt, rows, cols, nx)
    w, xs, y0 = wide_case_inputs(fmt, rows, cols, nx, seed)
    assert bytes(G[f"w{i}_digest"]) == digest(w, xs, y0)
    st = col_stride_floats(cols)
    dx, _ = dev_cols(flh, gpu, xs, st)
    flh.act_q8(dx, cols, gpu, nx=nx, xstride=st)
    dy = flh.DeviceBuffer.from_array(y0, gpu)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    flh.stream_dot(fmt, dw, rows, cols, dx, dy, gpu, nx=nx, xstride=st, ystride=rows)
    got = dy.download(np.float32, y0.size, gpu)
    assert np.array_equal(bits(got), bits(G[f"w{i}_y"]))
    if nx == 1 and fmt != 1:
        # the fused ACT_Q8 + STREAM_DOT launch gives the same bits
        dx2, _ = dev_cols(flh, gpu, xs, st)
        dy2 = flh.DeviceBuffer.from_array(y0, gpu)
        flh.act_q8_stream_dot(fmt, dw, rows, cols, dx2, dy2, gpu)
        assert np.array_equal(bits(dy2.download(np.float32, y0.size, gpu)), bits(G[f"w{i}_y"]))


def test_device_q8_0_quantizer_equals_reference_q8_1_blocks(flh, gpu):
    rows, cols, seed = Q8_0_QUANT
    say("q8_0 quantizer", rows, cols)
    wf = (np.random.default_rng(seed).standard_normal((rows, cols)) * 0.02).astype(np.float32)
    src = flh.DeviceBuffer.from_array(wf.ravel(), gpu)
    dst = flh.DeviceBuffer(G["q80_bytes"].size)
    flh.quantize(1, src, rows, cols, dst, gpu)
    got = dst.download(np.uint8, G["q80_bytes"].size, gpu).reshape(rows, -1)
    assert np.array_equal(got, G["q80_bytes"])
