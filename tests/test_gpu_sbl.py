"""GPU parity of the superblock-per-lane single-column Q4_K kernel
(fast-llm_amd/csrc/flh_dot_sbl.hip), which serves every single-column Q4_K
STREAM_DOT with at most 64 superblocks per row.

Bar: bitwise against the oracle (fl_dot_i8k_q4_K, src/runtime/quants.h:538-561)
for every chunk geometry (rows per chunk = 64 // superblocks per row, partial
last chunks, idle lanes), both workgroup widths, one or two workgroups per CU,
grids so small that a wave's chunk list outgrows one batch of preloaded old y
values, any number of waves requesting a chunk before the activation is
staged, with y += accumulation onto random y, and with ACT_Q8 fused (the
appendix bytes in memory must equal ACT_Q8's).
"""
import numpy as np
import pytest

from oracle import Q4_K, col_stride_floats, x_alloc_bytes
from util import tuned, sane_rows, normal_weights, activations
from test_gpu_parity import bits, say, dev_cols, run_dot

pytestmark = pytest.mark.gpu

# (rows, cols): superblocks per row 1, 2, 3, 5, 11, 16, 56, 64; rows that
# leave a partial last chunk
SHAPES = [(7, 256), (33, 512), (41, 768), (37, 1024), (29, 1280), (19, 2048), (13, 2816), (1001, 4096), (9, 14336),
          (70, 16384), (4096, 4096)]
CONFIGS = ["1,8,1,0", "1,4,1,0", "1,6,1,0,255", "1,4,2,0", "1,8,1,3,1", "1,4,1,1,255", "1"]


def fused_run(flh, orc, gpu, w, rows, cols, xs, y0):
    st = col_stride_floats(cols)
    dx, _ = dev_cols(flh, gpu, xs, st)
    dy = flh.DeviceBuffer.from_array(y0, gpu)
    dw = flh.DeviceBuffer.from_array(w, gpu)
    flh.act_q8_stream_dot(Q4_K, dw, rows, cols, dx, dy, gpu)
    got = dy.download(np.float32, rows, gpu)
    xq = dx.download(np.float32, st, gpu)
    ref_x = orc.act_q8_cols(xs, st)
    n = x_alloc_bytes(cols) // 4
    assert np.array_equal(xq[:n].view(np.uint8), ref_x[:n].view(np.uint8)), "appendix bytes"
    want = y0.copy()
    orc.stream_dot(Q4_K, w, rows, cols, ref_x, want, threads=8)
    return got, want


@pytest.mark.parametrize("cfg", CONFIGS)
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_sbl_bitwise(flh, orc, gpu, cfg, rows, cols):
    say("sbl", cfg, rows, cols)
    rng = np.random.default_rng(rows * 3 + cols)
    w = sane_rows(Q4_K, rows, cols, rng)
    xs = activations(1, cols, rng, outliers=True)
    y0 = rng.standard_normal(rows).astype(np.float32)
    with tuned(flh, FLH_SBL=cfg):
        got, want = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs, y0=y0)
        assert np.array_equal(bits(got), bits(want))
        got, want = fused_run(flh, orc, gpu, w, rows, cols, xs, y0)
        assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("rows,cols", [(6144, 4096), (4096, 14336), (16384, 4096), (6144, 8192)])
def test_sbl_layer_shapes_normal_weights(flh, orc, gpu, rows, cols):
    """Quantized N(0, 0.02^2) weights (the benchmark's recipe) at layer shapes."""
    say("sbl layer", rows, cols)
    rng = np.random.default_rng(rows + cols)
    w = flh.quantize_host(Q4_K, normal_weights(rows, cols, rng))
    xs = activations(1, cols, rng, outliers=True)
    y0 = np.zeros(rows, np.float32)
    got, want = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs, y0=y0)
    assert np.array_equal(bits(got), bits(want))
    got, want = fused_run(flh, orc, gpu, w, rows, cols, xs, y0)
    assert np.array_equal(bits(got), bits(want))


def test_sbl_matches_streaming_kernel(flh, orc, gpu):
    """The two single-column kernels give the same bits (FLH_SBL=0 runs the
    four-lanes-per-superblock streaming kernel)."""
    rows, cols = 3000, 4096
    rng = np.random.default_rng(11)
    w = sane_rows(Q4_K, rows, cols, rng)
    xs = activations(1, cols, rng)
    y0 = rng.standard_normal(rows).astype(np.float32)
    got1, want = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs, y0=y0)
    with tuned(flh, FLH_SBL="0"):
        got0, _ = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs, y0=y0)
    assert np.array_equal(bits(got1), bits(got0))
    assert np.array_equal(bits(got1), bits(want))


def test_wide_rows_both_kernels(flh, orc, gpu):
    """8192 x 14336 (56 superblocks per row, above 2^18 superblocks): the
    default launch goes to the streaming kernel, a forced FLH_SBL plan to this
    one; both bitwise against the oracle, unfused and with ACT_Q8 fused."""
    rows, cols = 8192, 14336
    say("wide rows", rows, cols)
    rng = np.random.default_rng(8192)
    w = flh.quantize_host(Q4_K, normal_weights(rows, cols, rng))
    xs = activations(1, cols, rng, outliers=True)
    y0 = rng.standard_normal(rows).astype(np.float32)
    for cfg in (None, "1,8,1,4"):
        with tuned(flh, **({} if cfg is None else {"FLH_SBL": cfg})):
            got, want = run_dot(flh, orc, gpu, Q4_K, w, rows, cols, xs, y0=y0)
            assert np.array_equal(bits(got), bits(want)), cfg
            got, want = fused_run(flh, orc, gpu, w, rows, cols, xs, y0)
            assert np.array_equal(bits(got), bits(want)), cfg


Q8_0 = 1


# rows of 8448-16128 columns (more than 64 four-block halves) put two halves
# on a lane; 16384 columns is past that plan and takes the other kernels
B32_SHAPES = [(7, 256), (33, 512), (41, 768), (13, 2816), (1001, 4096), (70, 8192), (4096, 4096), (37, 8448),
              (50, 14336), (9, 16128), (5, 16384)]


@pytest.mark.parametrize("cfg", ["1", "1,8,1,0", "1,4,2,0,255", "1,6,1,3,1"])
@pytest.mark.parametrize("rows,cols", B32_SHAPES)
def test_sbl_q8_0_bitwise(flh, orc, gpu, cfg, rows, cols):
    """Q8_0 x q8_1 with half a 256-weight unit per lane: bitwise
    fl_dot_i8_q8_0 (src/runtime/quants.h:438-447) for every unit count per
    row up to 63 (16128 columns; above 32, two halves per lane)."""
    say("sbl q8_0", cfg, rows, cols)
    rng = np.random.default_rng(rows * 5 + cols)
    w = sane_rows(Q8_0, rows, cols, rng)
    xs = activations(1, cols, rng, outliers=True)
    y0 = rng.standard_normal(rows).astype(np.float32)
    with tuned(flh, FLH_SBL=cfg):
        got, want = run_dot(flh, orc, gpu, Q8_0, w, rows, cols, xs, y0=y0)
        assert np.array_equal(bits(got), bits(want))


Q5_0, IQ2_XXS, IQ3_XXS = 2, 5, 6
B32_MODE = {Q8_0: "int8", Q5_0: "int8", IQ2_XXS: "iq8", IQ3_XXS: "iq8"}


@pytest.mark.parametrize("cfg", ["1", "1,8,1,0", "1,4,2,0,255", "1,6,1,3,1"])
@pytest.mark.parametrize("rows,cols", B32_SHAPES)
def test_sbl_q5_0_bitwise(flh, orc, gpu, cfg, rows, cols):
    """Q5_0 x q8_1 with 4 blocks (88 bytes) per lane: bitwise fl_dot_i8_q5_0
    (src/runtime/quants.h:449-466) for every lane count per row up to 64,
    and two halves per lane above that."""
    say("sbl q5_0", cfg, rows, cols)
    rng = np.random.default_rng(rows * 7 + cols)
    w = sane_rows(Q5_0, rows, cols, rng)
    xs = activations(1, cols, rng, outliers=True)
    y0 = rng.standard_normal(rows).astype(np.float32)
    with tuned(flh, FLH_SBL=cfg):
        got, want = run_dot(flh, orc, gpu, Q5_0, w, rows, cols, xs, y0=y0)
        assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", [IQ2_XXS, IQ3_XXS])
@pytest.mark.parametrize("cfg", ["1", "1,8,1,0", "1,4,2,0,255", "1,6,1,3,1"])
@pytest.mark.parametrize("rows,cols", [(5, 2048), (33, 2048), (1001, 4096), (70, 8192), (4096, 4096), (21, 10240),
                                       (50, 14336), (3, 16384)])
def test_sbl_iq_bitwise(flh, orc, gpu, fmt, cfg, rows, cols):
    """IQ2_XXS / IQ3_XXS x q8_1 with half a superblock per lane (2-byte
    aligned pieces, codebook staged in LDS): bitwise against the oracle's
    group order (fmaf(db * dx, idot, a[b & 3]))."""
    say("sbl iq", fmt, cfg, rows, cols)
    rng = np.random.default_rng(rows * 11 + cols + fmt)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(1, cols, rng, outliers=True)
    y0 = rng.standard_normal(rows).astype(np.float32)
    with tuned(flh, FLH_SBL=cfg):
        got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode="iq8", y0=y0)
        assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("rows,cols", [(14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("fmt", [Q8_0, Q5_0, IQ2_XXS, IQ3_XXS])
def test_sbl_b32_matches_register_kernel(flh, orc, gpu, fmt, rows, cols):
    """The LDS-staged and register kernels give the same bits (and both the
    oracle's) on a layer-sized matrix (4096x14336: two halves per lane) and
    on an expert picked by an id slot."""
    say("sbl b32 vs register", fmt, rows, cols)
    rng = np.random.default_rng(900 + fmt + cols)
    w = sane_rows(fmt, rows, cols, rng)
    xs = activations(1, cols, rng, outliers=True)
    outs = []
    for cfg in ("1", "0"):
        with tuned(flh, FLH_SBL=cfg):
            got, want = run_dot(flh, orc, gpu, fmt, w, rows, cols, xs, mode=B32_MODE[fmt])
            assert np.array_equal(bits(got), bits(want)), cfg
            outs.append(got)
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
    r, ne = 96, 3
    we = sane_rows(fmt, r * ne, cols, rng)
    got, want = run_dot(flh, orc, gpu, fmt, we, r, cols, xs, mode=B32_MODE[fmt], id_slot=1,
                        estride=r * flh.row_bytes(fmt, cols))
    assert np.array_equal(bits(got), bits(want))


Q6_K = 4


# (explicit wave counts: by default the launcher leaves Q6_K below vocab size
# to the streaming kernel)
@pytest.mark.parametrize("cfg", ["1,4,1,0", "1,8,1,0", "1,4,2,0,255", "1,6,1,3,1"])
@pytest.mark.parametrize("rows,cols", [(7, 2048), (33, 4096), (1001, 4096), (41, 6144), (13, 10240), (9, 14336),
                                       (70, 16384), (4096, 4096)])
def test_sbl_q6_k_bitwise(flh, orc, gpu, cfg, rows, cols):
    """Q6_K x q8_K with one 210-byte superblock per lane (2-byte aligned in
    LDS): bitwise fl_dot_i8k_q6_K (src/runtime/quants.h:563-594) for rows of
    8 and 16 superblocks (folded by DPP), 24 (parked in lane order) and 40,
    56, 64 (one row per chunk, chains parked contiguously)."""
    say("sbl q6_K", cfg, rows, cols)
    rng = np.random.default_rng(rows * 3 + cols)
    w = sane_rows(Q6_K, rows, cols, rng)
    xs = activations(1, cols, rng, outliers=True)
    y0 = rng.standard_normal(rows).astype(np.float32)
    with tuned(flh, FLH_SBL=cfg):
        got, want = run_dot(flh, orc, gpu, Q6_K, w, rows, cols, xs, y0=y0)
        assert np.array_equal(bits(got), bits(want))


def test_sbl_q6_k_matches_streaming_kernel(flh, orc, gpu):
    """Vocab-head Q6_K 65536x4096 (large enough for the default launch to
    take the superblock-per-lane kernel): it and the four-lanes-per-superblock
    kernel give the oracle's bits; and a zero activation gives +0.0 exactly
    (the parked second product adds nothing)."""
    say("sbl q6_K vs kstream")
    rng = np.random.default_rng(66)
    rows, cols = 65536, 4096
    w = sane_rows(Q6_K, rows, cols, rng)
    xs = activations(1, cols, rng, outliers=True)
    outs = []
    for cfg in ("1", "0"):
        with tuned(flh, FLH_SBL=cfg):
            got, want = run_dot(flh, orc, gpu, Q6_K, w, rows, cols, xs)
            assert np.array_equal(bits(got), bits(want)), cfg
            outs.append(got)
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
    with tuned(flh, FLH_SBL="1,4,1,0"):
        got, want = run_dot(flh, orc, gpu, Q6_K, w[:9 * flh.row_bytes(Q6_K, cols)], 9, cols,
                            np.zeros((1, cols), np.float32))
        assert np.array_equal(bits(got), bits(want))
