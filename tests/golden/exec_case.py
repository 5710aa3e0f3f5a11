"""Inputs of the run_serial fixture (tests/golden/exec_moe.npz): one token of a
MoE FFN with 4 experts, top-2, d 512, ff 768, from fixed seeds.  Shared by the
fixture writer (make_exec_golden.py) and the tests, which regenerate the same
bytes instead of storing ~1 MB of weights."""
import os
import sys

import numpy as np

_T = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, _T)
sys.path.insert(0, os.path.join(os.path.dirname(_T), "oracle"))
from util import sane_rows  # noqa: E402

D, FF, NE, TOPK = 512, 768, 4, 2
Q4_K, Q6_K = 3, 4


def inputs():
    rng = np.random.default_rng(20261202)
    x = rng.standard_normal(D).astype(np.float32)
    logits = rng.standard_normal(NE).astype(np.float32)
    wgu = sane_rows(Q4_K, NE * 2 * FF, D, rng)
    wdn = sane_rows(Q6_K, NE * D, FF, rng)
    return x, logits, wgu, wdn
