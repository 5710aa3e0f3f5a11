"""Writes tests/golden/exec_moe.npz: a frozen MoE FFN task table built with the
reference's own Arena / Graph and its outputs after the reference's run_serial
(src/runtime/graph.cpp:116-148), through oracle/_ref/libflref.so
(oracle/ref_shim.cpp: ref_run_serial_moe).  Run in the build container:
    python tests/golden/make_exec_golden.py
The fixture holds data only: the table bytes with every arena pointer
rewritten as an offset, the parameter structs, and the output bytes."""
import ctypes as C
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, HERE)
from exec_case import D, FF, NE, TOPK, inputs  # noqa: E402

NAMES = ["x", "logits", "ids", "gates", "wgu", "wdn", "gu", "h", "parts", "y", "router_p", "silu_p",
         "wmerge_p", "hstride"]


def main():
    lib = C.CDLL(os.path.join(ROOT, "oracle", "_ref", "libflref.so"))
    f = lib.ref_run_serial_moe
    f.restype = C.c_int
    x, logits, wgu, wdn = inputs()
    cap = 16 << 20
    pre = np.zeros(cap, np.uint8)
    post = np.zeros(cap, np.uint8)
    used = C.c_uint64()
    nt = C.c_uint32()
    off = (C.c_uint64 * 14)()
    P = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    rc = f(C.c_uint32(D), C.c_uint32(FF), C.c_uint32(NE), C.c_uint32(TOPK), P(x), P(logits), P(wgu), P(wdn),
           P(pre), P(post), C.c_size_t(cap), C.byref(used), C.byref(nt), off)
    assert rc == 0
    used, nt, off = used.value, nt.value, list(off)
    table = pre[:nt * 256].copy()
    # arena base = task 0's x minus the x offset (task 0 is ACT_Q8(x))
    L = json.load(open(os.path.join(HERE, "task_layout.json")))   # offsets read from the reference header
    t0x = int(table[L["x"]:L["x"] + 8].view(np.uint64)[0])
    base = t0x - off[0]

    def rel(v):
        return v - base if v else 0

    tab = table.reshape(nt, 256).copy()
    for i in range(nt):
        for o in (L["w"], L["x"], L["y"], L["aux"]):
            v = int(tab[i, o:o + 8].view(np.uint64)[0])
            tab[i, o:o + 8] = np.frombuffer(np.uint64(rel(v)).tobytes(), np.uint8)
    hs = off[13]

    def seg(a, o, n):
        return a[o:o + n].copy()
    pstructs = {"router_p": seg(pre, off[10], 40), "silu_p": seg(pre, off[11], 32 * TOPK),
                "wmerge_p": seg(pre, off[12], 56)}
    for k, v in pstructs.items():                          # pointer members -> offsets
        w = v.view(np.uint64)
        n_ptr = {"router_p": 3, "silu_p": None, "wmerge_p": 5}[k]
        idx = range(n_ptr) if n_ptr else [j for p in range(TOPK) for j in (4 * p, 4 * p + 1, 4 * p + 2)]
        for j in idx:
            w[j] = rel(int(w[j]))
    xalloc_d = off[2] - off[0]
    out = {
        "table": tab.ravel(), "offsets": np.array(off[:13], np.uint64), "used": np.uint64(used),
        "hstride": np.uint64(hs), **pstructs,
        "x_after": seg(post, off[0], xalloc_d),
        "ids": seg(post, off[2], 4 * TOPK), "gates": seg(post, off[3], 4 * TOPK),
        "gu": seg(post, off[6], 4 * TOPK * 2 * FF), "h": seg(post, off[7], 4 * hs * TOPK),
        "parts": seg(post, off[8], 4 * TOPK * D), "y": seg(post, off[9], 4 * D),
    }
    np.savez_compressed(os.path.join(HERE, "exec_moe.npz"), **out)
    print("wrote exec_moe.npz:", nt, "tasks,", used, "arena bytes")


if __name__ == "__main__":
    main()
