"""flh_exec_tasks runs a task table frozen by the reference itself and matches
the reference's run_serial (src/runtime/graph.cpp:116-148) on it.

tests/golden/exec_moe.npz holds a one-token MoE FFN graph built with the
reference's Arena / Graph (oracle/ref_shim.cpp: ref_run_serial_moe, written by
tests/golden/make_exec_golden.py): ACT_Q8, ROUTER_SEL, per routed slot two
gate/up STREAM_DOT_IDX row tiles, SILU_MUL, ACT_Q8, the down STREAM_DOT_IDX,
then WMERGE and SIGNAL, with the consumer lists and dep counts freeze()
computed.  The table is relocated into device memory as it is (every arena
pointer rebased; the op parameter structs stay host-side, where
flh_exec_tasks reads them) and executed in the canonical mode that run_serial
uses (exec_task_scalar).  Bar: the activation appendix, the expert ids and the
gate/up dots bit for bit; what follows the expf of the router and SILU
(gates, h, down dots, y) within the float tolerance of those ops (rtol
2e-6 on gates and h, 1e-5 of max |.| downstream), and bitwise wherever
the device expf rounds as the host's did."""
import ctypes as C
import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
from exec_case import D, FF, NE, TOPK, inputs  # noqa: E402

pytestmark = pytest.mark.gpu


def test_exec_tasks_matches_run_serial(flh, gpu):
    print("[case] run_serial fixture", flush=True)
    fx = np.load(os.path.join(ROOT, "tests", "golden", "exec_moe.npz"), allow_pickle=False)
    L = json.load(open(os.path.join(ROOT, "tests", "golden", "task_layout.json")))
    off = [int(v) for v in fx["offsets"]]
    used = int(fx["used"])
    x, logits, wgu, wdn = inputs()
    arena = flh.DeviceBuffer(used)
    arena.zero(gpu)
    for o, a in ((off[0], x), (off[1], logits), (off[4], wgu), (off[5], wdn)):
        arena.upload(np.ascontiguousarray(a), gpu, offset=o)
    dev = arena.ptr

    def reloc(v):
        return dev + v if v else 0

    # op parameter structs, host-side, their pointer members rebased
    keep = []

    def pstruct(cls, raw, nptr):
        b = bytearray(raw.tobytes())
        w = np.frombuffer(b, np.uint64)
        for j in range(nptr):
            w[j] = reloc(int(w[j]))
        s = cls.from_buffer_copy(bytes(b[:C.sizeof(cls)]))
        keep.append(s)
        return C.addressof(s)

    rp = pstruct(flh.RouterP, fx["router_p"], 3)
    sps = [pstruct(flh.SiluMulP, fx["silu_p"][32 * k:32 * k + 32], 3) for k in range(TOPK)]
    wp = pstruct(flh.WmergeP, fx["wmerge_p"], 5)
    aux_host = {off[10]: rp, off[12]: wp}
    for k in range(TOPK):
        aux_host[off[11] + 32 * k] = sps[k]

    tab = fx["table"].reshape(-1, 256)
    tasks = []
    for row in tab:
        t = flh.Task.from_buffer_copy(row.tobytes())
        for f in ("w", "x", "y"):
            setattr(t, f, reloc(getattr(t, f) or 0))
        a = t.aux or 0
        t.aux = aux_host[a] if a in aux_host else reloc(a)
        tasks.append(t)
    assert [int(t.kind) for t in tasks] == [3, 10, 4, 4, 11, 3, 4, 4, 4, 11, 3, 4, 12, 2]
    assert C.sizeof(flh.Task) == L["sizeof"]

    flh.exec_tasks(tasks, gpu, fast=False)
    gpu.sync()

    def get(o, n):
        return arena.download(np.uint8, n, gpu, offset=o)

    xa = fx["x_after"]
    n = flh.x_alloc_bytes(D)
    assert np.array_equal(get(off[0], n), xa[:n]), "ACT_Q8 appendix"
    assert np.array_equal(get(off[2], 4 * TOPK), fx["ids"]), "expert ids"
    g = get(off[3], 4 * TOPK).view(np.float32)
    np.testing.assert_allclose(g, fx["gates"].view(np.float32), rtol=2e-6)
    assert np.array_equal(get(off[6], 8 * TOPK * FF), fx["gu"]), "gate/up dots"
    hs = int(fx["hstride"])
    h = get(off[7], 4 * hs * TOPK).view(np.float32).reshape(TOPK, hs)[:, :FF]
    hw = fx["h"].view(np.float32).reshape(TOPK, hs)[:, :FF]
    np.testing.assert_allclose(h, hw, rtol=2e-6)
    parts = get(off[8], 4 * TOPK * D).view(np.float32)
    pw = fx["parts"].view(np.float32)
    assert np.max(np.abs(parts - pw)) <= 1e-5 * np.max(np.abs(pw))
    y = get(off[9], 4 * D).view(np.float32)
    yw = fx["y"].view(np.float32)
    assert np.max(np.abs(y - yw)) <= 1e-5 * np.max(np.abs(yw))
    print("bitwise: gates", np.array_equal(g, fx["gates"].view(np.float32)), "h", np.array_equal(h, hw),
          "parts", np.array_equal(parts, pw), "y", np.array_equal(y, yw), flush=True)
