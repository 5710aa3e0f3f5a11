"""The run_serial fixture (tests/golden/exec_moe.npz, written by the
reference's own Graph + run_serial, src/runtime/graph.cpp:116-148) agrees with
the oracle restatement step by step: the ACT_Q8 appendix bytes, the router's
ids and gates, the canonical gate/up dots of the routed experts, SILU_MUL,
the canonical down dots and WMERGE, all bit for bit.  This pins the fixture
(and the oracle) before the GPU test compares flh_exec_tasks with it."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
from exec_case import D, FF, NE, TOPK, Q4_K, Q6_K, inputs  # noqa: E402
from oracle import row_bytes  # noqa: E402


@pytest.fixture(scope="module")
def fx():
    return np.load(os.path.join(ROOT, "tests", "golden", "exec_moe.npz"), allow_pickle=False)


def f32(a):
    return a.view(np.float32)


def test_fixture_against_oracle(orc, fx):
    x, logits, wgu, wdn = inputs()
    xb = orc.act_q8(x)
    assert np.array_equal(fx["x_after"][:xb.nbytes], xb.view(np.uint8))
    ids, gates = orc.router_sel(logits, TOPK)
    assert np.array_equal(ids, fx["ids"].view(np.uint32))
    assert np.array_equal(gates.view(np.uint32), fx["gates"].view(np.uint32))
    rb4, rb6 = row_bytes(Q4_K, D), row_bytes(Q6_K, FF)
    hs = int(fx["hstride"])
    gu = f32(fx["gu"]).reshape(TOPK, 2 * FF)
    hh = f32(fx["h"]).reshape(TOPK, hs)
    parts = f32(fx["parts"]).reshape(TOPK, D)
    for k, e in enumerate(ids):
        want = np.zeros(2 * FF, np.float32)
        orc.stream_dot(Q4_K, wgu[e * 2 * FF * rb4:(e + 1) * 2 * FF * rb4], 2 * FF, D, xb.view(np.float32), want, fast=False, i8_mask=0, i8k_mask=0)
        assert np.array_equal(gu[k].view(np.uint32), want.view(np.uint32)), k
        h = orc.silu_mul(want[:FF], want[FF:])
        assert np.array_equal(hh[k, :FF].view(np.uint32), h.view(np.uint32)), k
        hb = orc.act_q8(h)
        assert np.array_equal(hh[k].view(np.uint8)[FF * 4:hb.nbytes], hb.view(np.uint8)[FF * 4:]), k
        pd = np.zeros(D, np.float32)
        orc.stream_dot(Q6_K, wdn[e * D * rb6:(e + 1) * D * rb6], D, FF, hb.view(np.float32), pd, fast=False, i8_mask=0, i8k_mask=0)
        assert np.array_equal(parts[k].view(np.uint32), pd.view(np.uint32)), k
    y = orc.wmerge(parts, gates, add1=x)
    assert np.array_equal(f32(fx["y"]).view(np.uint32), y.view(np.uint32))
