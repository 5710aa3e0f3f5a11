"""Write golden vectors from the reference's own CPU code.

Runs ONLY in the build container, where /root/reference exists:
  make -C oracle ref && python tests/golden/make_golden.py
It calls oracle/_ref/libflref.so (the reference's quants.h / kernels.h /
decode_params.h compiled from its sources by oracle/Makefile) on seeded
inputs and stores inputs + outputs as small .npz fixtures next to this file.
Input generation follows the reference tests' own recipes: random payload
bytes with sane fp16 scales (tests/test_quants.cpp:109-128,
tests/test_runtime.cpp:460-487) and x uniform in [-1, 1) (N(0,1), with
1 % x20 outliers, for some cases).
It also records the byte layout of fastllm::Task (include/fastllm/fastllm.h
:65-97) by compiling a 10-line offsetof probe against the reference header.
"""
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
from oracle import Oracle, row_bytes, col_stride_floats, F32, Q8_0, Q5_0, Q4_K, Q6_K  # noqa: E402

REF = "/root/reference"


def sane_rows(fmt, rows, cols, rng):
    """Random block bytes with finite fp16 scales (small positive halves)."""
    w = rng.integers(0, 256, size=rows * row_bytes(fmt, cols), dtype=np.uint8)
    bb = {Q8_0: 34, Q5_0: 22, Q4_K: 144, Q6_K: 210}[fmt]
    blocks = w.reshape(-1, bb)
    def half():
        return (0x2000 | (rng.integers(0, 1 << 16, size=blocks.shape[0]) & 0x0BFF)).astype(np.uint16)
    if fmt == Q6_K:
        blocks[:, 208:210] = half().view(np.uint8).reshape(-1, 2)
    else:
        blocks[:, 0:2] = half().view(np.uint8).reshape(-1, 2)
        if fmt == Q4_K:
            blocks[:, 2:4] = half().view(np.uint8).reshape(-1, 2)
    return w


def xs_for(cols, nx, rng, outliers=False):
    x = rng.uniform(-1, 1, size=(nx, cols)).astype(np.float32)
    if outliers:
        m = rng.random(size=x.shape) < 0.01
        x[m] *= 20.0
    return x


def task_layout():
    src = r'''
#include "fastllm/fastllm.h"
#include <cstddef>
#include <cstdio>
using fastllm::Task;
#define O(f) printf("\"%s\": %zu,\n", #f, offsetof(Task, f));
int main() { printf("{\n");
O(id) O(kind) O(affinity) O(fmt) O(n_consumers) O(consumers) O(w) O(w_bytes) O(x) O(y)
O(rows) O(cols) O(dep_init) O(dep_count) O(epoch) O(handoff_ts) O(aux) O(aux2) O(nx)
O(xstride) O(ystride)
printf("\"sizeof\": %zu, \"alignof\": %zu}\n", sizeof(Task), alignof(Task)); }
'''
    with tempfile.TemporaryDirectory() as d:
        cpp, exe = os.path.join(d, "p.cpp"), os.path.join(d, "p")
        open(cpp, "w").write(src)
        subprocess.check_call(["g++", "-std=c++17", "-I", REF + "/include", cpp, "-o", exe])
        return json.loads(subprocess.check_output([exe]).decode())


def main():
    ref = Oracle(ref=True)
    rng = np.random.default_rng(20261201)
    out = {}

    # ---- fp16 conversion: specials + random bit patterns
    specials = np.array([1.0, -2.0, 65504.0, 1e30, 5.96046448e-8, 0.0, -0.0, np.inf, -np.inf,
                         np.nan, 65519.0, 65520.0, 2.98e-8, 2.99e-8, 6.1035156e-05, 6.09e-05],
                        dtype=np.float32)
    rnd = rng.integers(0, 1 << 32, size=4000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    small = (rng.standard_normal(2000) * 1e-5).astype(np.float32)
    f = np.concatenate([specials, rnd, small]).astype(np.float32)
    out["f2h_in"] = f
    out["f2h_out"] = np.array([ref.float2half(float(v)) for v in f], dtype=np.uint16)

    # ---- ACT_Q8 appendices
    for cols, kind in [(96, "u"), (256, "n"), (512, "z"), (2816, "u"), (4096, "o")]:
        if kind == "n":
            x = rng.standard_normal(cols).astype(np.float32)
        elif kind == "z":
            x = rng.uniform(-1, 1, cols).astype(np.float32)
            x[32:64] = 0.0                      # an all-zero q8_1 block
            x[300:310] = 1e-40                  # denormals
        elif kind == "o":
            x = rng.standard_normal(cols).astype(np.float32)
            m = rng.random(cols) < 0.01
            x[m] *= 20.0
        else:
            x = rng.uniform(-1, 1, cols).astype(np.float32)
        out[f"act_{cols}_x"] = x
        out[f"act_{cols}_buf"] = ref.act_q8(x)

    # ---- dequant
    for fmt, cols in [(Q8_0, 512), (Q4_K, 1024), (Q6_K, 1024)]:
        w = sane_rows(fmt, 3, cols, rng)
        out[f"dq_{fmt}_w"] = w
        out[f"dq_{fmt}_out"] = ref.dequant(fmt, w, 3, cols)

    # ---- STREAM_DOT, every routing mode of exec_task_cpu
    modes = {  # name: (fast, i8_mask, i8k_mask)
        "i8k": (1, 0b11110, 0b11000), "i8": (1, 0b11110, 0), "f32fast": (1, 0, 0), "canon": (0, 0, 0)}
    cases = []
    for fmt, cols in [(Q8_0, 512), (Q8_0, 2816), (Q4_K, 512), (Q4_K, 2816), (Q6_K, 512), (Q6_K, 2816)]:
        for mode in ("i8k", "i8", "f32fast", "canon"):
            if mode == "i8k" and fmt == Q8_0:
                continue
            for nx in (1, 3):
                cases.append((fmt, cols, mode, nx))
    for i, (fmt, cols, mode, nx) in enumerate(cases):
        rows = 7
        w = sane_rows(fmt, rows, cols, rng)
        xs = xs_for(cols, nx, rng, outliers=(i % 3 == 0))
        st = col_stride_floats(cols)
        # build the column buffer with the REFERENCE's own ACT_Q8
        xbuf = np.zeros(nx * st, dtype=np.float32)
        for p in range(nx):
            col = ref.act_q8(xs[p])
            xbuf[p * st:p * st + col.size // 4] = col.view(np.float32)
        y0 = rng.standard_normal(nx * rows).astype(np.float32)
        y = y0.copy()
        fast, i8, i8k = modes[mode]
        ref.stream_dot(fmt, w, rows, cols, xbuf, y, nx=nx, xstride=st, ystride=rows,
                       fast=fast, i8_mask=i8, i8k_mask=i8k)
        key = f"dot{i}"
        out[key + "_meta"] = np.array([fmt, cols, rows, nx, st, fast, i8, i8k], dtype=np.int64)
        out[key + "_w"], out[key + "_x"], out[key + "_y0"], out[key + "_y"] = w, xbuf, y0, y
    out["dot_count"] = np.array([len(cases)])

    # STREAM_DOT_IDX: expert 2 of 3
    rows, cols = 5, 1024
    we = sane_rows(Q4_K, 3 * rows, cols, rng)
    xs = xs_for(cols, 1, rng)
    st = col_stride_floats(cols)
    xbuf = np.zeros(st, dtype=np.float32)
    col = ref.act_q8(xs[0])
    xbuf[:col.size // 4] = col.view(np.float32)
    y = np.zeros(rows, dtype=np.float32)
    ref.stream_dot(Q4_K, we, rows, cols, xbuf, y, fast=1, i8_mask=0b11110, i8k_mask=0b11000,
                   id_slot=2, estride=rows * row_bytes(Q4_K, cols))
    out.update({"idx_w": we, "idx_x": xbuf, "idx_y": y})

    # ---- MoE glue
    kat = np.array([0.1, 2.0, -1.0, 2.0, 0.5, 1.9, -3.0, 0.0], dtype=np.float32)
    out["router_kat_in"] = kat
    for norm in (0, 1):
        ids, gates = ref.router_sel(kat, 3, norm=norm, scale=1.0)
        out[f"router_kat_ids_{norm}"], out[f"router_kat_gates_{norm}"] = ids, gates
    logits = rng.standard_normal((16, 8)).astype(np.float32)
    out["router_in"] = logits
    rid, rg = zip(*[ref.router_sel(l, 2, norm=1, scale=1.0) for l in logits])
    out["router_ids"], out["router_gates"] = np.stack(rid), np.stack(rg)
    g = (rng.uniform(-1, 1, 4096) * 4).astype(np.float32)
    u = rng.uniform(-1, 1, 4096).astype(np.float32)
    out.update({"silu_g": g, "silu_u": u, "silu_h": ref.silu_mul(g, u)})
    parts = rng.standard_normal((2, 4096)).astype(np.float32)
    gates = np.array([0.7, 0.3], dtype=np.float32)
    add1 = rng.standard_normal(4096).astype(np.float32)
    out.update({"wm_parts": parts, "wm_gates": gates, "wm_add1": add1,
                "wm_y": ref.wmerge(parts, gates, add1=add1, scale=1.0)})

    # ---- Q5_0 (own RNG stream, so the cases above keep their bytes): dequant
    # and every STREAM_DOT routing mode; cols 1408 = 5.5 chunks of 256 also
    # covers the fast path's partial last dequant chunk (kernels.h:244-254)
    rng5 = np.random.default_rng(20261202)
    w = sane_rows(Q5_0, 3, 1408, rng5)
    out["dq5_w"], out["dq5_out"] = w, ref.dequant(Q5_0, w, 3, 1408)
    n5 = 0
    for cols in (512, 1408):
        for mode in ("i8", "f32fast", "canon"):
            for nx in (1, 3):
                rows = 7
                w = sane_rows(Q5_0, rows, cols, rng5)
                xs = xs_for(cols, nx, rng5, outliers=(n5 % 2 == 0))
                st = col_stride_floats(cols)
                xbuf = np.zeros(nx * st, dtype=np.float32)
                for p in range(nx):
                    col = ref.act_q8(xs[p])
                    xbuf[p * st:p * st + col.size // 4] = col.view(np.float32)
                y0 = rng5.standard_normal(nx * rows).astype(np.float32)
                y = y0.copy()
                fast, i8, i8k = modes[mode]
                ref.stream_dot(Q5_0, w, rows, cols, xbuf, y, nx=nx, xstride=st, ystride=rows,
                               fast=fast, i8_mask=i8, i8k_mask=i8k)
                key = f"q5dot{n5}"
                out[key + "_meta"] = np.array([Q5_0, cols, rows, nx, st, fast, i8, i8k], dtype=np.int64)
                out[key + "_w"], out[key + "_x"], out[key + "_y0"], out[key + "_y"] = w, xbuf, y0, y
                n5 += 1
    out["q5dot_count"] = np.array([n5])

    # ---- IQ2_XXS / IQ3_XXS: the reference runs them on its CPU only through
    # the canonical chain (fl_dot_row_iq2_xxs / fl_dot_row_iq3_xxs,
    # quants.h:237-290); its fast / int8 CPU routes have no codebook case.
    # Canonical dots of random blocks (every grid index and sign pattern
    # occurs), the reference KAT block (tests/test_runtime.cpp:979-993), and
    # digests of the reference's codebooks and sign table.
    rngq = np.random.default_rng(20261203)
    nq = 0
    for fmt, bb in ((5, 66), (6, 98)):
        for cols, rows, nx in ((256, 64, 1), (2048, 9, 2), (512, 40, 3)):
            w = rngq.integers(0, 256, size=rows * (cols // 256) * bb, dtype=np.uint8)
            blocks = w.reshape(-1, bb)
            blocks[:, 0:2] = (0x2000 | (rngq.integers(0, 1 << 16, blocks.shape[0]) & 0x0BFF)
                              ).astype(np.uint16).view(np.uint8).reshape(-1, 2)
            xs = xs_for(cols, nx, rngq, outliers=(nq % 2 == 1))
            st = col_stride_floats(cols)
            xbuf = np.zeros(nx * st, dtype=np.float32)
            for p in range(nx):
                xbuf[p * st:p * st + cols] = xs[p]
            y0 = rngq.standard_normal(nx * rows).astype(np.float32)
            y = y0.copy()
            ref.stream_dot(fmt, w, rows, cols, xbuf, y, nx=nx, xstride=st, ystride=rows,
                           fast=False, i8_mask=0, i8k_mask=0)
            key = f"iqdot{nq}"
            out[key + "_meta"] = np.array([fmt, cols, rows, nx, st, 0, 0, 0], dtype=np.int64)
            out[key + "_w"], out[key + "_x"], out[key + "_y0"], out[key + "_y"] = w, xbuf, y0, y
            nq += 1
    out["iqdot_count"] = np.array([nq])
    kat = np.zeros(66, dtype=np.uint8)
    kat[0:2] = np.array([0x3C00], dtype=np.uint16).view(np.uint8)
    xk = np.zeros(256, dtype=np.float32)
    xk[3] = 2.0
    yk = np.zeros(1, dtype=np.float32)
    ref.stream_dot(5, kat, 1, 256, xk, yk, fast=False, i8_mask=0, i8k_mask=0)
    out["iq_kat_w"], out["iq_kat_x"], out["iq_kat_y"] = kat, xk, yk
    import hashlib
    g2 = np.zeros(256, dtype=np.uint64)
    g3 = np.zeros(256, dtype=np.uint32)
    sg = np.zeros(128, dtype=np.uint8)
    import ctypes
    ref.lib.ref_iq_tables.argtypes = [ctypes.c_void_p] * 3
    ref.lib.ref_iq_tables(g2.ctypes.data, g3.ctypes.data, sg.ctypes.data)
    out["iq_sha256"] = np.array([hashlib.sha256(a.tobytes()).hexdigest() for a in (g2, g3, sg)])

    np.savez_compressed(os.path.join(HERE, "golden_ref.npz"), **out)
    with open(os.path.join(HERE, "task_layout.json"), "w") as fh:
        json.dump(task_layout(), fh, indent=1, sort_keys=True)
    print("wrote", os.path.join(HERE, "golden_ref.npz"),
          os.path.getsize(os.path.join(HERE, "golden_ref.npz")), "bytes")


if __name__ == "__main__":
    main()
