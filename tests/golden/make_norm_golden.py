"""Golden vectors of RMSNORM and of the decoder's norm -> quant -> matvec
chain from the reference's own CPU code.

Runs ONLY in the build container, where /root/reference exists:
  make -C oracle ref && python tests/golden/make_norm_golden.py
For every NORM_CASES input (tests/norm_cases.py) it stores the digest of the
inputs and fl_op_rmsnorm's y (src/runtime/decode_params.h:101-106).  For
every CHAIN_CASES input it runs the chain of src/model/decoder.cpp:874-880
on the reference's functions: fl_op_rmsnorm, fl_exec_act_q8 of its output
(src/runtime/quants.h:404-416), then exec_task_cpu's STREAM_DOT with the CPU
default masks (the q8_K int8 dot fl_dot_i8k_q4_K, quants.h:538-561), and
stores the normed column, its appendix bytes and the dot.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
from oracle import Oracle, Q4_K  # noqa: E402
from norm_cases import NORM_CASES, CHAIN_CASES, EPS, norm_inputs, chain_inputs, digest  # noqa: E402


def main():
    ref = Oracle(ref=True)
    out = {}
    for i, (n, seed, osc) in enumerate(NORM_CASES):
        x, wn = norm_inputs(n, seed, osc)
        out[f"n{i}_digest"] = np.frombuffer(digest(x, wn), dtype=np.uint8)
        out[f"n{i}_y"] = ref.rmsnorm(x, wn, EPS)
        print(f"norm case {i}: n {n}")
    for i, (rows, cols, seed) in enumerate(CHAIN_CASES):
        x, wn, w = chain_inputs(rows, cols, seed)
        yn = ref.rmsnorm(x, wn, EPS)
        col = ref.act_q8(yn)
        y = np.zeros(rows, dtype=np.float32)
        ref.stream_dot(Q4_K, w, rows, cols, col.view(np.float32), y, fast=1, i8_mask=0b11110, i8k_mask=0b11000)
        out[f"c{i}_digest"] = np.frombuffer(digest(x, wn, w), dtype=np.uint8)
        out[f"c{i}_col"] = col
        out[f"c{i}_y"] = y
        print(f"chain case {i}: {rows}x{cols}")
    np.savez_compressed(os.path.join(HERE, "golden_norm.npz"), **out)


if __name__ == "__main__":
    main()
