"""The persistent plan executor (flh_plan_*) against flh_exec_tasks and the oracle.

A decoder layer's task table is built the way the reference's graph builder
builds it (src/model/decoder.cpp:482-543, 607-634, 874-906): ACT_Q8 ->
row-tiled STREAM_DOTs, tiles fanned in to the next ACT_Q8, fan-out through
SIGNAL relay trees when a producer has more than kMaxConsumers (6)
consumers (decoder.cpp:552-605), SILU_MUL -> ACT_Q8 -> down tiles, a SIGNAL
sink.  The plan runs the whole table in one launch and must reproduce
flh_exec_tasks (which is bitwise equal to the reference CPU path, see
test_gpu_tasks / test_gpu_parity) bit for bit: every output, the
intermediate SILU_MUL output and every appendix byte -- on repeated launches,
and on replays of a captured HIP graph.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import Q4_K, Q6_K, Q8_0, col_stride_floats, row_bytes
from util import activations

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


class Graph:
    """Task table with the reference's edge rules (Graph::add / edge)."""

    def __init__(self, flh):
        self.flh, self.tasks, self.keep = flh, [], []

    def add(self, kind, **kw):
        t = self.flh.Task()
        t.kind = int(kind)
        for k, v in kw.items():
            setattr(t, k, v)
        self.tasks.append(t)
        return len(self.tasks) - 1

    def edge(self, p, c):
        t = self.tasks[p]
        assert t.n_consumers < 6
        t.consumers[t.n_consumers] = c
        t.n_consumers += 1

    def fan_out(self, p, consumers):
        """p -> every consumer, through SIGNAL relays appended at the end."""
        if len(consumers) <= 6:
            for c in consumers:
                self.edge(p, c)
            return
        relays = []
        for i in range(0, len(consumers), 6):
            r = self.add(self.flh.TaskKind.SIGNAL)
            for c in consumers[i:i + 6]:
                self.edge(r, c)
            relays.append(r)
        self.fan_out(p, relays)


class Layer:
    """Device buffers of one decoder layer's matvec chain."""

    def __init__(self, flh, gpu, fmt, D, F, qkv, rng, tile=256):
        self.flh, self.gpu, self.fmt, self.D, self.F, self.qkv, self.tile = flh, gpu, fmt, D, F, qkv, tile
        stD, stF = col_stride_floats(D), col_stride_floats(F)
        self.stD, self.stF = stD, stF
        xs = activations(3, D, rng, outliers=True)
        xb = np.zeros(3 * stD, np.float32)
        for p in range(3):
            xb[p * stD:p * stD + D] = xs[p]
        self.x = flh.DeviceBuffer.from_array(xb, gpu)
        self.shapes = {"qkv": (qkv, D), "o": (D, D), "gu": (2 * F, D), "dn": (D, F)}
        self.w = {}
        for name, (r, c) in self.shapes.items():
            self.w[name] = self.weights(r, c, rng)
        self.y = {n: flh.DeviceBuffer(4 * r) for n, (r, c) in self.shapes.items()}
        self.h = flh.DeviceBuffer(4 * stF)
        self.silu = flh.SiluMulP()

    def weights(self, rows, cols, rng):
        flh, gpu = self.flh, self.gpu
        w = flh.DeviceBuffer(rows * row_bytes(self.fmt, cols))
        stage = flh.DeviceBuffer(4 * cols * min(rows, 1024))
        for r0 in range(0, rows, 1024):
            n = min(1024, rows - r0)
            flh.fill_normal(stage, n * cols, int(rng.integers(1 << 30)), gpu, std=0.02)
            flh.quantize(self.fmt, stage, n, cols, w.ptr + r0 * row_bytes(self.fmt, cols), gpu)
        gpu.sync()
        stage.close()
        return w

    def xcol(self, p):
        return self.x.ptr + 4 * p * self.stD

    def reset(self):
        for b in self.y.values():
            b.zero(self.gpu)
        self.h.zero(self.gpu)
        self.gpu.sync()

    def table(self, edges=True):
        flh, T = self.flh, self.flh.TaskKind
        g = Graph(flh)
        D, F = self.D, self.F

        def act(x, cols):
            return g.add(T.ACT_Q8, x=x, y=x + flh.xq_offset(cols), rows=cols // 32, cols=cols)

        def tiles(name, x):
            r, c = self.shapes[name]
            rb = row_bytes(self.fmt, c)
            out = []
            for r0 in range(0, r, self.tile):
                n = min(self.tile, r - r0)
                out.append(g.add(T.STREAM_DOT, fmt=self.fmt, w=self.w[name].ptr + r0 * rb, w_bytes=n * rb,
                                 x=x, y=self.y[name].ptr + 4 * r0, rows=n, cols=c))
            return out

        a0 = act(self.xcol(0), D)
        t_qkv = tiles("qkv", self.xcol(0))
        a1 = act(self.xcol(1), D)              # stands in for attention: O waits for QKV
        t_o = tiles("o", self.xcol(1))
        a2 = act(self.xcol(2), D)              # stands in for residual + norm
        t_gu = tiles("gu", self.xcol(2))
        self.silu.gate = self.y["gu"].ptr
        self.silu.up = self.y["gu"].ptr + 4 * F
        self.silu.h = self.h.ptr
        self.silu.n = F
        s = g.add(T.SILU_MUL, aux=C.addressof(self.silu), rows=F, cols=1)
        a3 = act(self.h.ptr, F)
        t_dn = tiles("dn", self.h.ptr)
        sink = g.add(T.SIGNAL)
        if edges:
            g.fan_out(a0, t_qkv)
            for t in t_qkv:
                g.edge(t, a1)
            g.fan_out(a1, t_o)
            for t in t_o:
                g.edge(t, a2)
            g.fan_out(a2, t_gu)
            for t in t_gu:
                g.edge(t, s)
            g.edge(s, a3)
            g.fan_out(a3, t_dn)
            for t in t_dn:
                g.edge(t, sink)
        return g.tasks

    def snapshot(self):
        gpu = self.gpu
        out = {n: b.download(np.uint32, b.nbytes // 4, gpu) for n, b in self.y.items()}
        out["h"] = self.h.download(np.uint32, self.h.nbytes // 4, gpu)
        out["x"] = self.x.download(np.uint32, self.x.nbytes // 4, gpu)
        return out


def assert_same(a, b, what):
    for k in a:
        assert np.array_equal(a[k], b[k]), f"{what}: {k} differs"


def run_both(flh, gpu, L, edges=True, reps=2):
    tasks = L.table(edges)
    L.reset()
    flh.exec_tasks(tasks, gpu)
    gpu.sync()
    want = L.snapshot()
    for k in ("qkv", "o", "gu", "dn", "h"):
        assert np.count_nonzero(want[k]) > want[k].size // 2, f"{k}: reference run left zeros"
    plan = flh.Plan(tasks)
    info = plan.info()
    for r in range(reps):
        L.reset()
        plan.launch(gpu)
        gpu.sync()
        assert_same(L.snapshot(), want, f"plan launch {r}")
    plan.status()
    return plan, want, info


@pytest.mark.parametrize("fmt", [Q4_K, Q6_K])
def test_plan_layer_matches_exec_tasks(flh, gpu, fmt):
    say("plan layer", fmt)
    L = Layer(flh, gpu, fmt, D=1024, F=2816, qkv=1536, rng=np.random.default_rng(fmt))
    plan, want, info = run_both(flh, gpu, L)
    assert info["ops"] >= 5 and info["grid"] > 0
    plan.close()


def test_plan_layer_oracle_spot_check(flh, orc, gpu):
    """The QKV output of a plan launch equals the oracle's reference-order dot."""
    say("plan oracle")
    rng = np.random.default_rng(11)
    L = Layer(flh, gpu, Q4_K, D=1024, F=1024, qkv=768, rng=rng)
    plan = flh.Plan(L.table())
    L.reset()
    plan.launch(gpu)
    gpu.sync()
    x0 = L.x.download(np.float32, L.stD, gpu)
    xq = orc.act_q8_cols(x0[None, :1024], L.stD)
    assert np.array_equal(x0.view(np.uint32)[:len(xq)], xq.view(np.uint32))
    w = L.w["qkv"].download(np.uint8, L.w["qkv"].nbytes, gpu)
    want = np.zeros(768, np.float32)
    orc.stream_dot(Q4_K, w, 768, 1024, xq, want)
    got = L.y["qkv"].download(np.float32, 768, gpu)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    plan.close()


def test_plan_without_edges_runs_in_order(flh, gpu):
    say("plan no edges")
    L = Layer(flh, gpu, Q4_K, D=512, F=1024, qkv=768, rng=np.random.default_rng(5))
    plan, _, _ = run_both(flh, gpu, L, edges=False)
    plan.close()


def test_plan_graph_replays(flh, gpu):
    """Capture the zeroing + one plan launch; replays with eager work between."""
    say("plan graph")
    L = Layer(flh, gpu, Q4_K, D=1024, F=2816, qkv=1536, rng=np.random.default_rng(6))
    tasks = L.table()
    L.reset()
    flh.exec_tasks(tasks, gpu)
    gpu.sync()
    want = L.snapshot()
    plan = flh.Plan(tasks)
    with flh.Graph.capture(gpu) as g:
        for b in L.y.values():
            b.zero(gpu)
        L.h.zero(gpu)
        plan.launch(gpu)
    for r in range(4):
        g.launch()
        gpu.sync()
        assert_same(L.snapshot(), want, f"replay {r}")
        L.reset()                        # eager work between replays
    g.close()
    plan.status()
    plan.close()


def test_plan_llama3_8b_layer(flh, gpu):
    """Full Llama-3-8B layer shapes (QKV 6144x4096, O 4096^2, gate/up
    28672x4096, down 4096x14336): plan == exec_tasks bitwise."""
    say("plan llama3-8b layer")
    L = Layer(flh, gpu, Q4_K, D=4096, F=14336, qkv=6144, rng=np.random.default_rng(7), tile=512)
    plan, _, info = run_both(flh, gpu, L, reps=3)
    assert info["lds_bytes"] <= 80 * 1024
    plan.close()


def test_plan_rejects_what_it_cannot_run(flh, gpu):
    say("plan unsupported")
    T = flh.TaskKind
    L = Layer(flh, gpu, Q4_K, D=512, F=512, qkv=256, rng=np.random.default_rng(8))
    base = L.table()

    def expect_unsupported(tasks):
        with pytest.raises(flh.FlhError) as e:
            flh.Plan(tasks)
        assert e.value.code == flh.ERR_UNSUPPORTED

    t = flh.Task()
    t.kind = int(T.ROUTER_SEL)
    t.aux = C.addressof(L.silu)          # any host block: rejected before it is read
    expect_unsupported(base + [t])
    q8 = flh.Task()
    q8.kind, q8.fmt, q8.rows, q8.cols = int(T.STREAM_DOT), Q8_0, 1, 512
    q8.w, q8.w_bytes, q8.x, q8.y = L.w["o"].ptr, row_bytes(Q8_0, 512), L.xcol(0), L.y["o"].ptr
    expect_unsupported(base + [q8])
    mixed = flh.Task()
    mixed.kind, mixed.fmt, mixed.rows, mixed.cols = int(T.STREAM_DOT), Q6_K, 1, 512
    mixed.w, mixed.w_bytes, mixed.x, mixed.y = L.w["o"].ptr, row_bytes(Q6_K, 512), L.xcol(0), L.y["o"].ptr
    expect_unsupported(base + [mixed])
    with pytest.raises(flh.FlhError):
        flh.Plan(base, fast=False)
