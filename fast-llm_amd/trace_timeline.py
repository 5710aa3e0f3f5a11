"""Per-wave timeline of the superblock-per-lane launches (development measurement).

Loads the library's trace build, in which every wave of k_dot_sbl writes
s_memrealtime stamps (100 MHz) at fixed points, and prints for each launch
shape the spread of those stamps relative to the launch's first wave:

  entry            the wave starts
  x landed         its activation loads (q8_K blocks, or the fp32 column) are in LDS
  quantised        (fused ACT_Q8) its share of the column is quantised
  staged           the workgroup's activation barrier has passed
  first chunk      its first weight chunk has landed
  last chunk       its last weight chunk has landed
  exit             its stores are acknowledged

Build the trace library first (in-tree, next to the product library):
  make -C fast-llm_amd/csrc EXTRA=-DFLH_TRACE OUT=../_trace/libfastllm_hip.so BUILD=../_trace/_build
then run (one GPU):
  python fast-llm_amd/trace_timeline.py
The product library is never replaced: the trace build is loaded from its own
path and only by this script.
"""
import ctypes as C
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
TRACE_LIB = os.path.join(HERE, "_trace", "libfastllm_hip.so")
Q4_K, Q8_0 = 3, 1
# (name, format, rows, cols, fused ACT_Q8)
SHAPES = [("o", Q4_K, 4096, 4096, False), ("o_fused", Q4_K, 4096, 4096, True),
          ("qkv", Q4_K, 6144, 4096, False), ("qkv_fused", Q4_K, 6144, 4096, True),
          ("down", Q4_K, 4096, 14336, False), ("gate_up", Q4_K, 28672, 4096, False),
          ("q8_0", Q8_0, 4096, 4096, False)]
STAMPS = [(0, "entry"), (5, "x landed"), (6, "quantised"), (1, "staged"), (2, "first chunk"),
          (3, "last chunk"), (4, "exit")]


def main():
    if not os.path.exists(TRACE_LIB):
        sys.exit(f"trace library missing: {TRACE_LIB} (see this file's docstring for the make line)")
    sys.path.insert(0, ROOT)
    import __graft_entry__ as ge
    flh = ge._pkg()
    flh.LIB_PATH = TRACE_LIB
    lib = flh.lib()
    lib.flh_sbl_trace.argtypes = [C.c_void_p, C.c_size_t]
    spec = importlib.util.spec_from_file_location("bench", os.path.join(ROOT, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    flh.init(0)
    s = flh.Stream()
    B = bench.Bench(flh, s)
    staging = B.buf(256 << 20)
    host = np.zeros(4096 * 64, dtype=np.uint64)
    print("| launch | us per launch (graph) | waves with chunks | " +
          " | ".join(f"{lab} p10 / med / p90 (us)" for _, lab in STAMPS) + " |")
    print("|---" * (3 + len(STAMPS)) + "|")
    for name, fmt, r, c, fused in SHAPES:
        nb = flh.row_bytes(fmt, c) * r
        ws = B.weights(fmt, r, c, bench.copies_for(nb), seed=5 + r, staging=staging)
        x, _ = B.activation(c, 1, 3, outliers=fmt == Q4_K)
        y = B.buf(r * 4)
        y.zero(s)

        def issue(i):
            if fused:
                flh.act_q8_stream_dot(fmt, ws[i % len(ws)], r, c, x, y, s)
            else:
                flh.stream_dot(fmt, ws[i % len(ws)], r, c, x, y, s)

        host[:] = 0
        s.sync()
        if lib.flh_sbl_trace_clear() != 0:                # stamps of an earlier shape's waves
            sys.exit("trace clear failed")
        us = B.time_graph(issue, 32)
        s.sync()
        lib.flh_sbl_trace(host.ctypes.data, host.size)
        t = host.reshape(-1, 8).astype(np.int64)
        t = t[t[:, 0] > 0]
        rel = (t[:, :7] - t[:, 0].min()) / 100.0
        busy = t[:, 7] > 0
        cells = []
        for k, _ in STAMPS:
            v = rel[busy, k] if k in (2, 3) else rel[:, k]
            if (t[:, k] == 0).all():
                cells.append("-")
                continue
            cells.append(f"{np.percentile(v, 10):.2f} / {np.median(v):.2f} / {np.percentile(v, 90):.2f}")
        print(f"| {name} {r}x{c} | {us:.2f} | {int(busy.sum())} of {len(t)} | " + " | ".join(cells) + " |",
              flush=True)
        del ws


if __name__ == "__main__":
    main()
