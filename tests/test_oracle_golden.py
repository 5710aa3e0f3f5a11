"""The C oracle reproduces the reference's own outputs bit for bit.

Fixtures: tests/golden/golden_ref.npz, written by tests/golden/make_golden.py
from the reference's quants.h / kernels.h / decode_params.h compiled in the
build container (oracle/_ref).  Every comparison here is bitwise.
"""
import numpy as np
import pytest

from oracle import x_alloc_bytes


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_float2half_matches_reference(orc, golden):
    f, h = golden["f2h_in"], golden["f2h_out"]
    got = np.array([orc.float2half(float(v)) for v in f], dtype=np.uint16)
    assert np.array_equal(got, h)


@pytest.mark.parametrize("cols", [96, 256, 512, 2816, 4096])
def test_act_q8_matches_reference(orc, golden, cols):
    x = golden[f"act_{cols}_x"]
    want = golden[f"act_{cols}_buf"]
    got = orc.act_q8(x)
    assert got.size == x_alloc_bytes(cols)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("fmt,cols", [(1, 512), (3, 1024), (4, 1024)])
def test_dequant_matches_reference(orc, golden, fmt, cols):
    w = golden[f"dq_{fmt}_w"]
    want = golden[f"dq_{fmt}_out"]
    got = orc.dequant(fmt, w, 3, cols)
    assert np.array_equal(bits(got), bits(want))


def test_stream_dot_every_mode_matches_reference(orc, golden):
    n = int(golden["dot_count"][0])
    assert n >= 40
    for i in range(n):
        fmt, cols, rows, nx, st, fast, i8, i8k = (int(v) for v in golden[f"dot{i}_meta"])
        y = golden[f"dot{i}_y0"].copy()
        orc.stream_dot(fmt, golden[f"dot{i}_w"], rows, cols, golden[f"dot{i}_x"], y, nx=nx,
                       xstride=st, ystride=rows, fast=fast, i8_mask=i8, i8k_mask=i8k)
        assert np.array_equal(bits(y), bits(golden[f"dot{i}_y"])), (i, fmt, cols, nx, fast, i8, i8k)


def test_q5_0_dequant_and_dots_match_reference(orc, golden):
    """Q5_0: bit-exact dequant and every routing mode (q8_1 int8, fast fp32
    with a partial last 256-chunk, canonical) vs the reference's own code."""
    got = orc.dequant(2, golden["dq5_w"], 3, 1408)
    assert np.array_equal(bits(got), bits(golden["dq5_out"]))
    n = int(golden["q5dot_count"][0])
    assert n == 12
    for i in range(n):
        fmt, cols, rows, nx, st, fast, i8, i8k = (int(v) for v in golden[f"q5dot{i}_meta"])
        y = golden[f"q5dot{i}_y0"].copy()
        orc.stream_dot(fmt, golden[f"q5dot{i}_w"], rows, cols, golden[f"q5dot{i}_x"], y, nx=nx,
                       xstride=st, ystride=rows, fast=fast, i8_mask=i8, i8k_mask=i8k)
        assert np.array_equal(bits(y), bits(golden[f"q5dot{i}_y"])), (i, cols, nx, fast, i8)


def test_stream_dot_idx_matches_reference(orc, golden):
    from oracle import row_bytes
    y = np.zeros(5, dtype=np.float32)
    orc.stream_dot(3, golden["idx_w"], 5, 1024, golden["idx_x"], y, fast=1,
                   id_slot=2, estride=5 * row_bytes(3, 1024))
    assert np.array_equal(bits(y), bits(golden["idx_y"]))


def test_router_kat(orc, golden):
    # tests/test_decode_ops.cpp:84-102: ties -> lower index first
    for norm in (0, 1):
        ids, gates = orc.router_sel(golden["router_kat_in"], 3, norm=norm)
        assert list(ids) == [1, 3, 5]
        assert np.array_equal(ids, golden[f"router_kat_ids_{norm}"])
        assert np.array_equal(bits(gates), bits(golden[f"router_kat_gates_{norm}"]))
    ids, gates = orc.router_sel(golden["router_kat_in"], 3, norm=1)
    assert abs(float(gates.sum()) - 1.0) < 1e-6


def test_router_silu_wmerge_match_reference(orc, golden):
    for t in range(golden["router_in"].shape[0]):
        ids, gates = orc.router_sel(golden["router_in"][t], 2, norm=1)
        assert np.array_equal(ids, golden["router_ids"][t])
        assert np.array_equal(bits(gates), bits(golden["router_gates"][t]))
    h = orc.silu_mul(golden["silu_g"], golden["silu_u"])
    assert np.array_equal(bits(h), bits(golden["silu_h"]))
    y = orc.wmerge(golden["wm_parts"], golden["wm_gates"], add1=golden["wm_add1"])
    assert np.array_equal(bits(y), bits(golden["wm_y"]))


def test_iq_codebooks_match_reference(orc, golden):
    """The IQ2_XXS / IQ3_XXS grids and the sign widening equal the
    reference's tables (src/model/iq_tables.h), compared by SHA-256."""
    import hashlib
    g2 = np.array([orc.iq2_grid(i) for i in range(256)], dtype=np.uint64)
    g3 = np.array([orc.iq3_grid(i) for i in range(256)], dtype=np.uint32)
    sg = np.array([orc.iq_signs(i) for i in range(128)], dtype=np.uint8)
    got = [hashlib.sha256(a.tobytes()).hexdigest() for a in (g2, g3, sg)]
    assert got == [str(v) for v in golden["iq_sha256"]]


def test_iq_canonical_dots_match_reference(orc, golden):
    """fl_dot_row_iq2_xxs / fl_dot_row_iq3_xxs (quants.h:237-290) through the
    canonical route, and the reference KAT block (test_runtime.cpp:979-993)."""
    n = int(golden["iqdot_count"][0])
    assert n == 6
    for i in range(n):
        fmt, cols, rows, nx, st, fast, i8, i8k = (int(v) for v in golden[f"iqdot{i}_meta"])
        y = golden[f"iqdot{i}_y0"].copy()
        orc.stream_dot(fmt, golden[f"iqdot{i}_w"], rows, cols, golden[f"iqdot{i}_x"], y, nx=nx,
                       xstride=st, ystride=rows, fast=False)
        assert np.array_equal(bits(y), bits(golden[f"iqdot{i}_y"])), (i, fmt, cols, nx)
    y = np.zeros(1, dtype=np.float32)
    orc.stream_dot(5, golden["iq_kat_w"], 1, 256, golden["iq_kat_x"], y, fast=False)
    assert y[0] == golden["iq_kat_y"][0] == 2.0


# ---- BASELINE widths (tests/golden/golden_wide.npz, inputs regenerated from seeds)
def _wide():
    import os
    return np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_wide.npz"))


def test_wide_inputs_regenerate_bit_for_bit():
    """The seeded generator still yields the bytes the reference saw."""
    from wide_cases import WIDE_CASES, wide_case_inputs, digest
    g = _wide()
    assert int(g["wide_count"][0]) == len(WIDE_CASES)
    for i, case in enumerate(WIDE_CASES):
        assert list(g[f"w{i}_meta"]) == list(case)
        w, xs, y0 = wide_case_inputs(*case)
        assert bytes(g[f"w{i}_digest"]) == digest(w, xs, y0), i


@pytest.mark.parametrize("i", range(11))
def test_oracle_wide_dots_match_reference(orc, i):
    """Int8 STREAM_DOT at the Llama-3-8B widths (4096 / 14336 columns, 1-8
    columns): the oracle equals the reference bit for bit."""
    from oracle import col_stride_floats
    from wide_cases import WIDE_CASES, wide_case_inputs
    g = _wide()
    fmt, rows, cols, nx, seed = WIDE_CASES[i]
    w, xs, y0 = wide_case_inputs(fmt, rows, cols, nx, seed)
    st = col_stride_floats(cols)
    y = y0.copy()
    orc.stream_dot(fmt, w, rows, cols, orc.act_q8_cols(xs, st), y, nx=nx, xstride=st, ystride=rows, threads=8)
    assert np.array_equal(bits(y), bits(g[f"w{i}_y"]))


def test_q8_0_weight_quantizer_matches_reference_q8_1_blocks(flh):
    """The library's Q8_0 weight quantizer (host path) writes the reference's
    q8_1 block bytes without s (fl_quantize_q8_1_block, quants.h:360-378)."""
    from wide_cases import Q8_0_QUANT
    g = _wide()
    rows, cols, seed = Q8_0_QUANT
    wf = (np.random.default_rng(seed).standard_normal((rows, cols)) * 0.02).astype(np.float32)
    got = flh.quantize_host(1, wf).reshape(rows, -1)
    assert np.array_equal(got, g["q80_bytes"])
