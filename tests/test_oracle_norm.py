"""orc_rmsnorm and the decoder's norm -> quant -> matvec chain reproduce the
reference's own outputs bit for bit.

Fixture: tests/golden/golden_norm.npz, written by
tests/golden/make_norm_golden.py from the reference's fl_op_rmsnorm
(src/runtime/decode_params.h:101-106), fl_exec_act_q8 and exec_task_cpu
compiled in the build container (oracle/_ref); inputs regenerated from the
seeds in tests/norm_cases.py and checked against the stored digests.
"""
import os

import numpy as np
import pytest

from oracle import Q4_K, REF_SO
from norm_cases import NORM_CASES, CHAIN_CASES, EPS, norm_inputs, chain_inputs, digest

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_norm.npz"))


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("i", range(len(NORM_CASES)))
def test_rmsnorm_matches_reference(orc, i):
    n, seed, osc = NORM_CASES[i]
    x, wn = norm_inputs(n, seed, osc)
    assert bytes(G[f"n{i}_digest"]) == digest(x, wn)
    assert np.array_equal(bits(orc.rmsnorm(x, wn, EPS)), bits(G[f"n{i}_y"]))


@pytest.mark.parametrize("i", range(len(CHAIN_CASES)))
def test_norm_chain_matches_reference(orc, i):
    """RMSNORM -> ACT_Q8 of its output -> Q4_K int8 dot, all on the oracle:
    the normed column, its appendices and the dot are the reference's bytes."""
    rows, cols, seed = CHAIN_CASES[i]
    x, wn, w = chain_inputs(rows, cols, seed)
    assert bytes(G[f"c{i}_digest"]) == digest(x, wn, w)
    col = orc.act_q8(orc.rmsnorm(x, wn, EPS))
    assert np.array_equal(col, G[f"c{i}_col"])
    y = np.zeros(rows, np.float32)
    orc.stream_dot(Q4_K, w, rows, cols, col.view(np.float32), y)
    assert np.array_equal(bits(y), bits(G[f"c{i}_y"]))


@pytest.mark.skipif(not os.path.exists(REF_SO), reason="oracle/_ref not built (no reference tree here)")
@pytest.mark.parametrize("n", [1, 7, 256, 4096, 14336, 16384])
def test_rmsnorm_matches_reference_live(orc, n):
    """The same against the reference's code run now, at more sizes and with
    extreme inputs (huge outliers, subnormal-scale entries, zeros)."""
    from oracle import Oracle
    ref = Oracle(ref=True)
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    x[rng.random(n) < 0.02] *= np.float32(1e4)
    x[rng.random(n) < 0.02] *= np.float32(1e-30)
    x[rng.random(n) < 0.02] = 0
    wn = rng.standard_normal(n).astype(np.float32)
    assert np.array_equal(bits(orc.rmsnorm(x, wn, EPS)), bits(ref.rmsnorm(x, wn, EPS)))
