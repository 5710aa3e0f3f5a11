"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/fastllm_hip.h declares, mirrors the reference Task layout, validates
arguments like Graph::freeze(), and never reaches for the oracle."""
import json
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = open(os.path.join(ROOT, "include", "fastllm_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(flh_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol(flh):
    L = flh.lib()
    names = header_functions()
    assert len(names) >= 35
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # and the Python binding declares a signature for each of them
    assert set(names) <= set(flh._SIGS), set(names) - set(flh._SIGS)


def test_task_layout_matches_reference(flh):
    ref = json.load(open(os.path.join(ROOT, "tests", "golden", "task_layout.json")))
    T = flh.Task
    assert C_sizeof(T) == ref["sizeof"] == 256
    for f, off in ref.items():
        if f in ("sizeof", "alignof"):
            continue
        assert getattr(T, f).offset == off, f


def C_sizeof(t):
    import ctypes
    return ctypes.sizeof(t)


def test_helpers_match_reference_layout(flh):
    L = flh.lib()
    for cols in (32, 256, 2816, 4096, 14336):
        assert L.flh_x_alloc_bytes(cols) == flh.x_alloc_bytes(cols)
        for fmt in (1, 3, 4):
            assert L.flh_row_bytes(fmt, cols - cols % 256 or 256) == flh.row_bytes(fmt, cols - cols % 256 or 256)
    i8, i8k = (flh.C.c_uint32() if hasattr(flh, "C") else None), None
    import ctypes
    a, b = ctypes.c_uint32(), ctypes.c_uint32()
    L.flh_default_masks(ctypes.byref(a), ctypes.byref(b))
    assert a.value == flh.I8_MASK_DEFAULT and b.value == flh.I8K_MASK_DEFAULT


def test_validation_mirrors_freeze(flh):
    """graph.cpp:84-90: block multiple, w_bytes, IDX slot/stride -- checked
    before any device work, so they hold without a GPU."""
    L = flh.lib()
    p = 1 << 20   # any aligned non-null address: validation fails before use
    rc = L.flh_stream_dot(3, p, 144 * 3, 3, 300, p, p, 1, 0, 0, None, 0, 1, 0, 0, None)
    assert rc == flh.ERR_ARG and b"multiple" in L.flh_last_error()
    rc = L.flh_stream_dot(3, p, 144 * 3 + 1, 3, 256, p, p, 1, 0, 0, None, 0, 1, 0, 0, None)
    assert rc == flh.ERR_ARG and b"w_bytes" in L.flh_last_error()
    rc = L.flh_stream_dot(3, p, 144 * 3, 3, 256, p, p, 1, 0, 0, p, 0, 1, 0, 0, None)
    assert rc == flh.ERR_ARG and b"IDX" in L.flh_last_error()
    rc = L.flh_stream_dot(3, p, 144 * 3, 3, 256, p, p, 17, 0, 0, None, 0, 1, 0, 0, None)
    assert rc == flh.ERR_ARG
    rc = L.flh_stream_dot(3, p + 2, 144 * 3, 3, 256, p, p, 1, 0, 0, None, 0, 1, 0, 0, None)
    assert rc == flh.ERR_ARG and b"aligned" in L.flh_last_error()
    # 2-byte aligned block formats take weights at any even address (row tiles
    # of rows 2 mod 4 bytes long), never at an odd one
    rc = L.flh_stream_dot(1, p + 1, 34 * 8 * 3, 3, 256, p, p, 1, 0, 0, None, 0, 1, 0, 0, None)
    assert rc == flh.ERR_ARG and b"aligned" in L.flh_last_error()
    rc = L.flh_stream_dot(1, p + 2, 34 * 8 * 3, 3, 256, p, p, 1, 0, 0, None, 0, 1, 0, 0, None)
    assert rc in (flh.ERR_STATE, flh.OK)
    # several columns whose outputs overlap (ystride < rows) would race on the device
    rc = L.flh_stream_dot(3, p, 144 * 3, 3, 256, p, p, 2, 2048, 2, None, 0, 1, 0, 0, None)
    assert rc == flh.ERR_ARG and b"overlap" in L.flh_last_error()
    # several activation columns closer than one column's allocation (fp32 + appendices)
    rc = L.flh_act_q8_stream_dot(3, p, 144 * 3, 3, 256, p, p, 2, 256, 3, None, 0, 1, 0, 0, None)
    assert rc == flh.ERR_ARG and b"overlap" in L.flh_last_error()
    # valid arguments but no flh_init -> state error, never a silent no-op
    rc = L.flh_stream_dot(3, p, 144 * 3, 3, 256, p, p, 1, 0, 0, None, 0, 1, 0, 0, None)
    assert rc in (flh.ERR_STATE, flh.OK)


def test_exec_tasks_rejects_unsupported_kinds(flh):
    t = flh.Task()
    t.kind = flh.TaskKind.ATTN_HEAD
    t.aux = 1 << 20
    arr = (flh.Task * 1)(t)
    import ctypes
    rc = flh.lib().flh_exec_tasks(ctypes.cast(arr, ctypes.c_void_p), 1, 1, 0, 0, None)
    assert rc == flh.ERR_UNSUPPORTED
    t.kind = flh.TaskKind.STREAM_DOT_IDX
    t.fmt, t.rows, t.cols, t.w, t.x, t.y = 3, 2, 256, 1 << 20, 1 << 20, 1 << 20
    t.w_bytes = 288
    t.aux, t.aux2 = 1 << 20, 0
    arr = (flh.Task * 1)(t)
    rc = flh.lib().flh_exec_tasks(ctypes.cast(arr, ctypes.c_void_p), 1, 1, 0, 0, None)
    assert rc == flh.ERR_ARG


def test_product_never_loads_the_oracle():
    for dirpath, _, files in os.walk(os.path.join(ROOT, "fast-llm_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".h", "Makefile")):
                txt = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in txt.lower() or f == "__init__.py" and "oracle" not in re.sub(
                    r'""".*?"""', "", txt, flags=re.S).lower(), f


def test_host_quantizer_round_trip(flh, orc):
    """Own weight quantizers (the reference has none): dequant(quant(w)) is
    close to w and every block decodes through the reference formulas."""
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((16, 1024)) * 0.02).astype(np.float32)
    for fmt, tol in ((1, 0.01), (3, 0.12), (4, 0.05)):
        q = flh.quantize_host(fmt, w)
        assert q.size == 16 * flh.row_bytes(fmt, 1024)
        d = orc.dequant(fmt, q, 16, 1024)
        rel = np.linalg.norm(d - w) / np.linalg.norm(w)
        assert rel < tol, (fmt, rel)
