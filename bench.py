"""Benchmark of the quantized decode hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): Q4_K matvec throughput at the
Llama-3-8B layer shapes, N=1.  One "step" = one decoder layer's four
STREAM_DOTs with their ACT_Q8 prologues, weights resident in HBM:
  ACT_Q8(x 4096) + QKV 6144x4096, ACT_Q8(x 4096) + O 4096x4096,
  ACT_Q8(x 4096) + gate/up 28672x4096, ACT_Q8(h 14336) + down 4096x14336.
Steps rotate over L layer copies (L * 122.7 MB > 2x the 256 MB Infinity
Cache) so HBM, not MALL, is measured.  The L layer steps are captured in
one HIP graph, as a decode step would run its layers: the timed region is
one launch of a graph of K layer steps (step i on copy i % L), bracketed
by stream syncs and HIP events; the W warmup steps are a graph of their own.  value = weight bytes streamed / second (GB/s, 1e9).

Also reported (same JSON line):
  ops      -- per-op us and GB/s for every BASELINE config: Q8_0 4096^2,
              each Q4_K layer shape, Q6_K vocab head and down, spec-verify
              N in {2,4,8}, MoE top-2 of 8 at batch 1 and 8 (graph of R
              launches rotating over weight copies, HIP events); also Q5_0 /
              IQ2_XXS / IQ3_XXS matvecs, 2/4/8-column dots of those formats
              and Q8_0 at 14336x4096, the activation quantisers
              (ACT_Q8 14336, RMSNORM -> ACT_Q8 4096) and RMSNORM -> QKV /
              gate/up in one launch against two, and the decoder's whole
              norm -> matvec chain of a layer (5 launches);
  roofline -- the dominant kernel (Q4_K gate/up): algorithmic bytes per
              launch / average launch time vs the 8 TB/s HBM peak;
  cpu_baseline -- the reference CPU path on the host cores (oracle/_ref,
              the reference's own code, if built; else the C restatement).
Inputs are synthetic: weights N(0, 0.02^2) quantized on the device, x
N(0,1) with 1 % x20 outliers for Q4_K.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
METRIC = "Q4_K/Q6_K matvec GB/s (% of HBM peak) + us/op at Llama-3-8B shapes, N=1"

Q8_0, Q5_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS = 1, 2, 3, 4, 5, 6
BLOCK = {Q5_0: (32, 22), IQ2_XXS: (256, 66), IQ3_XXS: (256, 98)}
LAYER = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)]


def col_stride(flh, cols):
    return ((flh.x_alloc_bytes(cols) + 127) & ~127) // 4


class Bench:
    def __init__(self, flh, stream):
        self.flh, self.s = flh, stream
        self.bufs = []

    def buf(self, nbytes):
        b = self.flh.DeviceBuffer(nbytes)
        self.bufs.append(b)
        return b

    def weights(self, fmt, rows, cols, copies, seed, staging):
        """`copies` quantized matrices of N(0, 0.02^2) weights, made on the device."""
        flh = self.flh
        rb = flh.row_bytes(fmt, cols)
        out = []
        for c in range(copies):
            w = self.buf(rows * rb)
            step = max(1, staging.nbytes // (cols * 4))
            for r0 in range(0, rows, step):
                nr = min(step, rows - r0)
                flh.fill_normal(staging, nr * cols, seed * 1000003 + c * 7919 + r0, self.s, std=0.02)
                flh.quantize(fmt, staging, nr, cols, w.ptr + r0 * rb, self.s)
            out.append(w)
        self.s.sync()
        return out

    def weights_random(self, fmt, rows, cols, copies, seed):
        """`copies` device copies of one matrix of random block bytes whose
        fp16 scale d (bytes 0-1 of each block) is finite, as the reference
        tests build them (tests/test_quants.cpp:109-128); the formats
        flh_quantize does not produce (Q5_0, IQ2_XXS, IQ3_XXS)."""
        rng = np.random.default_rng(seed)
        n, bb = BLOCK[fmt]
        w = rng.integers(0, 256, size=rows * (cols // n) * bb, dtype=np.uint8)
        blocks = w.reshape(-1, bb)
        d = (0x2000 | (rng.integers(0, 1 << 16, size=blocks.shape[0]) & 0x0BFF)).astype(np.uint16)
        blocks[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        out = [self.flh.DeviceBuffer.from_array(w, self.s) for _ in range(copies)]
        self.bufs.extend(out)
        self.s.sync()
        return out

    def activation(self, cols, nx, seed, outliers):
        st = col_stride(self.flh, cols)
        x = self.buf(nx * st * 4)
        x.zero(self.s)
        for p in range(nx):
            self.flh.fill_normal(x.ptr + p * st * 4, cols, seed + p, self.s,
                                 outlier_frac=0.01 if outliers else 0.0, outlier_scale=20.0)
        self.flh.act_q8(x, cols, self.s, nx=nx, xstride=st)
        return x, st

    def time_graph(self, issue, reps, replays=5):
        """Capture issue() `reps` times in one graph; return us per rep, the
        median over `replays` timed replays (after one untimed replay)."""
        flh = self.flh
        with flh.Graph.capture(self.s) as g:
            for i in range(reps):
                issue(i)
        g.launch()                      # warm
        self.s.sync()
        e0, e1 = flh.Event(), flh.Event()
        ts = []
        for _ in range(replays):
            e0.record(self.s)
            g.launch()
            e1.record(self.s)
            self.s.sync()
            ts.append(e0.elapsed_ms(e1) * 1e3 / reps)
        g.close()
        e0.close()
        e1.close()
        return sorted(ts)[len(ts) // 2]


def copies_for(nbytes):
    return max(2, -(-3 * MALL_BYTES // nbytes))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-ops", action="store_true", help="headline only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--profile", nargs="?", const="gate_up", choices=sorted(PROFILE_OPS) + [PROFILE_ALL],
                    help="counter-collection run: a 256 MiB device copy (calibration) and "
                         "64 launches of one operation only (see PROFILE_OPS), no JSON line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the matvec would shard by "
              "rows across GPUs; no multi-GPU path is built); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import __graft_entry__ as ge
    flh = ge._pkg()
    flh.init(0)
    info = flh.device_info()
    s = flh.Stream()
    B = Bench(flh, s)
    staging = B.buf(256 << 20)

    if args.profile:
        profile_run(flh, B, s, staging, args.profile)
        return

    # ------------------------------------------------ headline: layer step
    layer_bytes = sum(flh.row_bytes(Q4_K, c) * r for _, r, c in LAYER)
    L = max(2, -(-3 * MALL_BYTES // layer_bytes))
    W = {name: [] for name, _, _ in LAYER}
    for name, r, c in LAYER:
        W[name] = B.weights(Q4_K, r, c, L, seed=101 + r + 7 * c, staging=staging)
    xin = {name: B.activation(c, 1, 10 + i, outliers=True) for i, (name, r, c) in enumerate(LAYER)}
    yout = {name: B.buf(r * 4) for name, r, c in LAYER}
    for y in yout.values():
        y.zero(s)

    def issue_layer(l):
        # ACT_Q8 + STREAM_DOT per matrix (one fused launch each, same bytes)
        for name, r, c in LAYER:
            x, st = xin[name]
            flh.act_q8_stream_dot(Q4_K, W[name][l], r, c, x, yout[name], s)

    # A decode step runs every layer back to back: the K timed steps are one
    # captured graph of K layer steps in order, rotating over the L copies
    # (step i uses copy i % L), so every timed step is the same decode shape
    # and one launch covers them; the W warmup steps are a graph of their own.
    def steps_graph(k):
        with flh.Graph.capture(s) as g:
            for i in range(k):
                issue_layer(i % L)
        return g

    timed = steps_graph(args.steps)
    warm = steps_graph(args.warmup) if args.warmup > 0 else None

    if warm is not None:
        warm.launch()
    s.sync()
    e0, e1 = flh.Event(), flh.Event()
    t0 = time.perf_counter()
    e0.record(s)
    timed.launch()
    e1.record(s)
    s.sync()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1)
    ms_per_step = ms / args.steps
    value = layer_bytes * args.steps / (ms * 1e-3) / 1e9

    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (weights N(0,0.02^2) quantized on device; x N(0,1), 1% x20 outliers)",
        "config": {"workload": "Llama-3-8B layer Q4_K matvecs, N=1 (BASELINE configs[1])",
                   "format": "Q4_K", "n": 1,
                   "shapes": {n: [r, c] for n, r, c in LAYER},
                   "weight_bytes_per_step": layer_bytes, "layer_copies": L,
                   "device": info["arch"], "cus": info["num_cus"]},
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "wall_s_timed": round(wall, 4),
    }

    # ------------------------------------------------- per-op measurements
    ops = {}

    def op_entry(name, us, wbytes, extra=None):
        e = {"us": round(us, 3), "weight_bytes": wbytes, "GBs": round(wbytes / us / 1e3, 1),
             "pct_hbm": round(100 * wbytes / us / 1e3 / HBM_PEAK_GBS, 2)}
        if extra:
            e.update(extra)
        ops[name] = e

    REPS = 64
    cpu_in = {}          # host copies of each config's bytes for the CPU baseline
    # The decoder's own chain over the same matrices (not the headline): the
    # attention norm + QKV in one launch, ACT_Q8 + O, the FFN norm + gate/up
    # in one launch, SILU_MUL + ACT_Q8 of the down input, down: 5 launches,
    # each depending on nothing but the previous in stream order.
    D_, F_ = 4096, 14336
    x0, _ = B.activation(D_, 1, 80, outliers=True)
    wn1, wn2 = B.buf(D_ * 4), B.buf(D_ * 4)
    flh.fill_normal(wn1, D_, 81, s, mean=1.0, std=0.1)
    flh.fill_normal(wn2, D_, 82, s, mean=1.0, std=0.1)
    xn1, _ = B.activation(D_, 1, 83, outliers=False)
    xn2, _ = B.activation(D_, 1, 84, outliers=False)
    h, _ = B.activation(F_, 1, 85, outliers=False)
    gu = yout["gate_up"]

    def chain(i):
        l = i % L
        flh.rmsnorm_stream_dot(Q4_K, W["qkv"][l], 6144, D_, x0, wn1, 1e-5, xn1, yout["qkv"], s)
        flh.act_q8_stream_dot(Q4_K, W["o"][l], D_, D_, xin["o"][0], yout["o"], s)
        flh.rmsnorm_stream_dot(Q4_K, W["gate_up"][l], 2 * F_, D_, x0, wn2, 1e-5, xn2, gu, s)
        flh.silu_mul_act_q8(gu, gu.ptr + F_ * 4, h, F_, 1, 2 * F_, col_stride(flh, F_), s)
        flh.stream_dot(Q4_K, W["down"][l], D_, F_, h, yout["down"], s)

    us = B.time_graph(chain, REPS)
    op_entry("decoder_chain_q4_K_layer", us, layer_bytes,
             {"launches": 5, "ops": "RMSNORM->ACT_Q8->QKV, ACT_Q8->O, RMSNORM->ACT_Q8->gate/up, "
                                    "SILU_MUL->ACT_Q8, down (one launch per arrow chain)"})
    for name, r, c in LAYER:
        x, st = xin[name]
        nb = r * flh.row_bytes(Q4_K, c)
        us = B.time_graph(lambda i: flh.stream_dot(Q4_K, W[name][i % L], r, c, x, yout[name], s), REPS)
        op_entry(f"q4_K_{name}_{r}x{c}", us, nb)
        if name != "down":
            # the fused ACT_Q8 + STREAM_DOT launch the layer step runs
            us = B.time_graph(lambda i: flh.act_q8_stream_dot(Q4_K, W[name][i % L], r, c, x, yout[name], s), REPS)
            op_entry(f"q4_K_{name}_{r}x{c}_act_fused", us, nb)
    # dominant kernel of the timed step: the fused ACT_Q8 + gate/up launch.
    # Algorithmic bytes: weights + fp32 x read + both appendices written
    # (by one workgroup) + y read and written.
    r, c = 28672, 4096
    gu = ops[f"q4_K_gate_up_{r}x{c}_act_fused"]
    alg = r * flh.row_bytes(Q4_K, c) + 4 * c + (c // 32) * 36 + (c // 256) * 292 + r * 8
    result["roofline"] = {"bound": "hbm", "achieved": round(alg / gu["us"] / 1e3, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(alg / gu["us"] / 1e3 / HBM_PEAK_GBS, 4),
                          "traffic": traffic_from_profile(),
                          "kernel": "k_dot_kstream<Q4_K,1,2,fused ACT_Q8,8 waves> gate/up 28672x4096 "
                                    "(the step's dominant launch)",
                          "alg_bytes_per_launch": alg, "us_per_launch": gu["us"]}

    if not args.no_ops:
        staging_cols = {}
        # Q6_K vocab head and down
        for name, r, c in [("vocab", 128256, 4096), ("down", 4096, 14336)]:
            nb = r * flh.row_bytes(Q6_K, c)
            ws = B.weights(Q6_K, r, c, copies_for(nb), seed=77 + r, staging=staging)
            x, st = B.activation(c, 1, 30, outliers=False)
            y = B.buf(r * 4)
            us = B.time_graph(lambda i: flh.stream_dot(Q6_K, ws[i % len(ws)], r, c, x, y, s),
                              8 if r > 100000 else REPS)
            op_entry(f"q6_K_{name}_{r}x{c}", us, nb)
            # the reference's GPU masks: Q6_K on the fast fp32 order
            us = B.time_graph(lambda i: flh.stream_dot(Q6_K, ws[i % len(ws)], r, c, x, y, s, i8_mask=0, i8k_mask=0),
                              4 if r > 100000 else 16)
            op_entry(f"q6_K_{name}_{r}x{c}_fast_f32", us, nb, {"route": "fast fp32 order (GPU default masks)"})
            cpu_in[f"q6_K_{name}_{r}x{c}"] = host_case(flh, s, Q6_K, ws[0], r, c, x, st, 1)
            if r > 100000:
                # a speculative-verify batch through the vocab head: 4, 8 and 16
                # columns in one weight pass (4: the streaming kernel, 8 and 16:
                # the Q6_K matrix-core kernel)
                for n in (4, 8, 16):
                    xn, stn = B.activation(c, n, 35 + n, outliers=False)
                    yn = B.buf(n * r * 4)
                    us = B.time_graph(lambda i: flh.stream_dot(Q6_K, ws[i % len(ws)], r, c, xn, yn, s, nx=n,
                                                               xstride=stn, ystride=r), 8)
                    op_entry(f"q6_K_vocab_verify_n{n}_{r}x{c}", us, nb, {"n": n})
                    del xn, yn
            del ws
        # Q6_K speculative verify at an FFN-up shape: 8 columns, four waves of
        # the matrix-core kernel per 32-row tile
        r, c = 14336, 4096
        nb = r * flh.row_bytes(Q6_K, c)
        ws = B.weights(Q6_K, r, c, copies_for(nb), seed=78, staging=staging)
        xn, stn = B.activation(c, 8, 43, outliers=False)
        yn = B.buf(8 * r * 4)
        us = B.time_graph(lambda i: flh.stream_dot(Q6_K, ws[i % len(ws)], r, c, xn, yn, s, nx=8, xstride=stn,
                                                   ystride=r), REPS)
        op_entry(f"q6_K_verify_n8_{r}x{c}", us, nb, {"n": 8})
        del ws
        # Q8_0
        r = c = 4096
        nb = r * flh.row_bytes(Q8_0, c)
        ws = B.weights(Q8_0, r, c, copies_for(nb), seed=5, staging=staging)
        x, st = B.activation(c, 1, 40, outliers=False)
        y = B.buf(r * 4)
        us = B.time_graph(lambda i: flh.stream_dot(Q8_0, ws[i % len(ws)], r, c, x, y, s), REPS)
        op_entry(f"q8_0_{r}x{c}", us, nb)
        cpu_in[f"q8_0_{r}x{c}"] = host_case(flh, s, Q8_0, ws[0], r, c, x, st, 1)
        del ws
        # the other 32-weight-block formats on the same kernel: Q5_0 and the
        # IQ codebook formats at an attention and an FFN shape (random
        # block bytes; the reference CPU path has no IQ int8 dot, so only
        # Q5_0 gets a CPU figure)
        for fmt, fname in ((Q5_0, "q5_0"), (IQ2_XXS, "iq2_xxs"), (IQ3_XXS, "iq3_xxs")):
            for r, c in ((4096, 4096), (14336, 4096)):
                nb = r * flh.row_bytes(fmt, c)
                ws = B.weights_random(fmt, r, c, copies_for(nb), seed=60 + fmt + r)
                y = B.buf(r * 4)
                # int8 dots for the IQ formats too (the reference's GPU default mask)
                m8 = flh.I8_MASK_DEFAULT | (1 << IQ2_XXS) | (1 << IQ3_XXS)
                us = B.time_graph(lambda i: flh.stream_dot(fmt, ws[i % len(ws)], r, c, x, y, s, i8_mask=m8), REPS)
                op_entry(f"{fname}_{r}x{c}", us, nb)
                if fmt == Q5_0 and r == 4096:
                    cpu_in[f"q5_0_{r}x{c}"] = host_case(flh, s, Q5_0, ws[0], r, c, x, st, 1)
                del ws
        # the down projection's shape (14336 columns: two four-block halves
        # per lane) in each 32-weight-block format
        x14, _ = B.activation(14336, 1, 41, outliers=False)
        for fmt, fname in ((Q8_0, "q8_0"), (Q5_0, "q5_0"), (IQ2_XXS, "iq2_xxs"), (IQ3_XXS, "iq3_xxs")):
            r, c = 4096, 14336
            nb = r * flh.row_bytes(fmt, c)
            ws = (B.weights(fmt, r, c, copies_for(nb), seed=61, staging=staging) if fmt == Q8_0
                  else B.weights_random(fmt, r, c, copies_for(nb), seed=62 + fmt))
            y = B.buf(r * 4)
            m8 = flh.I8_MASK_DEFAULT | (1 << IQ2_XXS) | (1 << IQ3_XXS)
            us = B.time_graph(lambda i: flh.stream_dot(fmt, ws[i % len(ws)], r, c, x14, y, s, i8_mask=m8), REPS)
            op_entry(f"{fname}_{r}x{c}", us, nb)
            del ws
        del x14
        # several activation columns of the 32-weight-block formats (a
        # speculative-verify batch on a Q8_0 / Q5_0 / IQ model): 14336x4096
        # with 2, 4, 8 columns, one weight pass per launch
        for fmt, fname in ((Q8_0, "q8_0"), (Q5_0, "q5_0"), (IQ2_XXS, "iq2_xxs"), (IQ3_XXS, "iq3_xxs")):
            r, c = 14336, 4096
            nb = r * flh.row_bytes(fmt, c)
            if fmt == Q8_0:
                ws = B.weights(fmt, r, c, copies_for(nb), seed=80 + r, staging=staging)
            else:
                ws = B.weights_random(fmt, r, c, copies_for(nb), seed=80 + fmt + r)
            m8 = flh.I8_MASK_DEFAULT | (1 << IQ2_XXS) | (1 << IQ3_XXS)
            for n in (2, 4, 8):
                xn, stn = B.activation(c, n, 90 + n, outliers=False)
                y = B.buf(n * r * 4)
                us = B.time_graph(lambda i: flh.stream_dot(fmt, ws[i % len(ws)], r, c, xn, y, s, nx=n, xstride=stn,
                                                           ystride=r, i8_mask=m8), REPS)
                op_entry(f"{fname}_verify_n{n}_{r}x{c}", us, nb, {"n": n})
            del ws
        # the activation quantisers on their own (row f1): ACT_Q8 of the
        # down projection's 14336-wide input (its own launch in the layer
        # step) and RMSNORM -> ACT_Q8 of a 4096-wide hidden state in one launch
        xq, _ = B.activation(14336, 1, 70, outliers=False)
        us = B.time_graph(lambda i: flh.act_q8(xq, 14336, s), REPS)
        op_entry("act_q8_14336", us, 14336 * 4 + 14336 // 32 * 36 + 14336 // 256 * 292,
                 {"bytes": "fp32 x read + both appendices written (no weights)"})
        xr, _ = B.activation(4096, 1, 71, outliers=False)
        wn = B.buf(4096 * 4)
        flh.fill_normal(wn, 4096, 72, s, mean=1.0, std=0.1)
        yr, _ = B.activation(4096, 1, 73, outliers=False)
        us = B.time_graph(lambda i: flh.rmsnorm_act_q8(xr, wn, yr, 4096, 1e-5, s), REPS)
        op_entry("rmsnorm_act_q8_4096", us, 3 * 4096 * 4 + 4096 // 32 * 36 + 4096 // 256 * 292,
                 {"bytes": "x and norm weight read, y and both appendices written (no matrix)"})
        # the decoder's norm -> quant -> matvec chain (attention norm -> QKV,
        # FFN norm -> gate/up): one launch (flh_rmsnorm_stream_dot) against
        # RMSNORM+ACT_Q8 and the dot as two launches
        for name, r, c in (("qkv", 6144, 4096), ("gate_up", 28672, 4096)):
            nb = r * flh.row_bytes(Q4_K, c)
            ws = B.weights(Q4_K, r, c, copies_for(nb), seed=74 + r, staging=staging)
            y = B.buf(r * 4)
            us = B.time_graph(lambda i: flh.rmsnorm_stream_dot(Q4_K, ws[i % len(ws)], r, c, xr, wn, 1e-5, yr, y, s),
                              REPS)
            op_entry(f"rmsnorm_q4_K_{name}_{r}x{c}_one_launch", us, nb)

            def two(i):
                flh.rmsnorm_act_q8(xr, wn, yr, c, 1e-5, s)
                flh.stream_dot(Q4_K, ws[i % len(ws)], r, c, yr, y, s)

            us = B.time_graph(two, REPS)
            op_entry(f"rmsnorm_q4_K_{name}_{r}x{c}_two_launches", us, nb)
            del ws
        # spec-verify small N
        for r, c in [(14336, 4096), (4096, 14336)]:
            nb = r * flh.row_bytes(Q4_K, c)
            ws = B.weights(Q4_K, r, c, copies_for(nb), seed=9 + r, staging=staging)
            for n in (2, 4, 8):
                x, st = B.activation(c, n, 50, outliers=True)
                y = B.buf(n * r * 4)
                us = B.time_graph(lambda i: flh.stream_dot(Q4_K, ws[i % len(ws)], r, c, x, y, s,
                                                           nx=n, xstride=st, ystride=r), REPS)
                op_entry(f"q4_K_verify_n{n}_{r}x{c}", us, nb, {"n": n})
                cpu_in[f"q4_K_verify_n{n}_{r}x{c}"] = host_case(flh, s, Q4_K, ws[0], r, c, x, st, n)
        # MoE decode: 8 experts, top-2, d_model 4096, d_ff 14336
        result["moe"] = bench_moe(flh, B, s, staging, cpu_in)
        ops.update(result["moe"].pop("ops"))
    result["ops"] = ops

    # ------------------------------------------------------- CPU baseline
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(flh, s, W, xin, cpu_in)
    print(json.dumps(result), flush=True)


# Operations a --profile run launches (64 times each, rotating over weight
# copies > 3x the Infinity Cache): name -> (format, rows, cols, columns, kind)
# kind: "dot" (STREAM_DOT on a ready appendix), "fused" (ACT_Q8 + STREAM_DOT
# in one launch), "act" (ACT_Q8 alone), "dot_nomfma" (the streaming kernel
# with the matrix-core kernel switched off).
PROFILE_OPS = {
    "gate_up": (Q4_K, 28672, 4096, 1, "dot"), "gate_up_fused": (Q4_K, 28672, 4096, 1, "fused"),
    "qkv": (Q4_K, 6144, 4096, 1, "dot"), "qkv_fused": (Q4_K, 6144, 4096, 1, "fused"),
    "o": (Q4_K, 4096, 4096, 1, "dot"), "o_fused": (Q4_K, 4096, 4096, 1, "fused"),
    "down": (Q4_K, 4096, 14336, 1, "dot"), "act_down": (Q4_K, 4096, 14336, 1, "act"),
    "q6k_vocab": (Q6_K, 128256, 4096, 1, "dot"), "q6k_down": (Q6_K, 4096, 14336, 1, "dot"),
    "q8_0": (Q8_0, 4096, 4096, 1, "dot"),
    "q8_0_down": (Q8_0, 4096, 14336, 1, "dot"), "q5_0_down": (Q5_0, 4096, 14336, 1, "dot"),
    "iq2_xxs_down": (IQ2_XXS, 4096, 14336, 1, "dot"), "iq3_xxs_down": (IQ3_XXS, 4096, 14336, 1, "dot"),
    "q5_0": (Q5_0, 4096, 4096, 1, "dot"), "q5_0_ffn": (Q5_0, 14336, 4096, 1, "dot"),
    "iq2_xxs": (IQ2_XXS, 4096, 4096, 1, "dot"), "iq2_xxs_ffn": (IQ2_XXS, 14336, 4096, 1, "dot"),
    "iq3_xxs": (IQ3_XXS, 4096, 4096, 1, "dot"), "iq3_xxs_ffn": (IQ3_XXS, 14336, 4096, 1, "dot"),
}
for _n in (2, 4, 8):
    for _r, _c in ((14336, 4096), (4096, 14336)):
        PROFILE_OPS[f"verify{_n}_{_r}x{_c}"] = (Q4_K, _r, _c, _n, "dot")
        PROFILE_OPS[f"verify{_n}_{_r}x{_c}_kstream"] = (Q4_K, _r, _c, _n, "dot_nomfma")
PROFILE_OPS["verify8"] = PROFILE_OPS["verify8_14336x4096"]
for _f, _name in ((Q8_0, "q8_0"), (Q5_0, "q5_0"), (IQ2_XXS, "iq2_xxs"), (IQ3_XXS, "iq3_xxs")):
    for _n in (2, 4, 8):
        PROFILE_OPS[f"{_name}_verify{_n}"] = (_f, 14336, 4096, _n, "dot")
PROFILE_OPS["q6k_vocab_verify8"] = (Q6_K, 128256, 4096, 8, "dot")
PROFILE_OPS["q6k_verify8_14336x4096"] = (Q6_K, 14336, 4096, 8, "dot")
PROFILE_OPS["q6k_vocab_f32fast"] = (Q6_K, 128256, 4096, 1, "dot_f32fast")
PROFILE_OPS["q6k_down_f32fast"] = (Q6_K, 4096, 14336, 1, "dot_f32fast")
PROFILE_OPS["norm_qkv"] = (Q4_K, 6144, 4096, 1, "norm")
PROFILE_OPS["norm_gate_up"] = (Q4_K, 28672, 4096, 1, "norm")


PROFILE_OPS["chain"] = (Q4_K, 0, 4096, 1, "chain")
PROFILE_OPS["moe1"] = (Q4_K, 0, 4096, 1, "moe")
PROFILE_OPS["moe8"] = (Q4_K, 0, 4096, 8, "moe")
PROFILE_OPS["act_q8_14336"] = (Q4_K, 0, 14336, 1, "act")
PROFILE_OPS["rmsnorm_act_q8"] = (Q4_K, 0, 4096, 1, "rmsnorm")
PROFILE_ALL = "all"


def profile_run(flh, B, s, staging, which="gate_up", launches=64, calibrate=True):
    """What the committed counter profiles were collected on: 5 device copies
    of 256 MiB (known HBM bytes: read 256 MiB + write 256 MiB each), then
    `launches` launches of one operation of PROFILE_OPS, issued straight on
    the stream (no graphs).  which="all": every operation of PROFILE_OPS in
    turn, 16 launches each (the kernel statistics of every bench op line)."""
    if calibrate:
        n = 256 << 20
        src, dst = B.buf(n), B.buf(n)
        src.zero(s)
        for _ in range(5):
            flh.copy(dst, src, n, s)
        s.sync()
    if which == PROFILE_ALL:
        for name in PROFILE_OPS:
            print(f"profile op {name}", flush=True)
            profile_run(flh, Bench(flh, s), s, staging, name, launches=16, calibrate=False)
        return
    fmt, r, c, nx, kind = PROFILE_OPS[which]
    if kind in ("chain", "moe", "act", "rmsnorm"):
        return profile_glue(flh, B, s, staging, kind, c, nx, launches)
    if kind == "dot_nomfma":
        os.environ["FLH_NO_MFMA"] = "1"
        flh.init(0)
    nb = r * flh.row_bytes(fmt, c)
    if fmt in BLOCK:
        ws = B.weights_random(fmt, r, c, copies_for(nb), seed=101 + r + 7 * c)
    else:
        ws = B.weights(fmt, r, c, copies_for(nb), seed=101 + r + 7 * c, staging=staging)
    x, st = B.activation(c, nx, 12, outliers=fmt == Q4_K)
    y = B.buf(nx * r * 4)
    m8 = flh.I8_MASK_DEFAULT | (1 << IQ2_XXS) | (1 << IQ3_XXS)
    if kind == "norm":                      # RMSNORM -> ACT_Q8 -> dot, one launch
        xn, _ = B.activation(c, 1, 13, outliers=False)
        wn = B.buf(c * 4)
        flh.fill_normal(wn, c, 14, s, mean=1.0, std=0.1)
    for i in range(launches):
        if kind == "norm":
            flh.rmsnorm_stream_dot(fmt, ws[i % len(ws)], r, c, x, wn, 1e-5, xn, y, s)
        elif kind == "fused":
            flh.act_q8_stream_dot(fmt, ws[i % len(ws)], r, c, x, y, s)
        elif kind == "dot_f32fast":         # the fast fp32 order (no int8 route)
            flh.stream_dot(fmt, ws[i % len(ws)], r, c, x, y, s, nx=nx, xstride=st, ystride=r, i8_mask=0, i8k_mask=0)
        else:
            flh.stream_dot(fmt, ws[i % len(ws)], r, c, x, y, s, nx=nx, xstride=st, ystride=r, i8_mask=m8)
    s.sync()
    if kind == "dot_nomfma":
        del os.environ["FLH_NO_MFMA"]
        flh.init(0)
    for b in B.bufs:
        b.close()
    B.bufs.clear()


def profile_glue(flh, B, s, staging, kind, cols, ntok, launches):
    """--profile runs of the op lines that are not one matvec: the decoder's
    5-launch chain of a layer, the MoE FFN (batch 1 or 8), ACT_Q8 of a
    14336-wide column, RMSNORM -> ACT_Q8 of a 4096-wide one."""
    if kind == "act":
        x, _ = B.activation(cols, 1, 70, outliers=False)
        for _ in range(launches):
            flh.act_q8(x, cols, s)
    elif kind == "rmsnorm":
        x, _ = B.activation(cols, 1, 71, outliers=False)
        wn = B.buf(cols * 4)
        flh.fill_normal(wn, cols, 72, s, mean=1.0, std=0.1)
        yr, _ = B.activation(cols, 1, 73, outliers=False)
        for _ in range(launches):
            flh.rmsnorm_act_q8(x, wn, yr, cols, 1e-5, s)
    elif kind == "chain":
        D_, F_ = 4096, 14336
        L = 3
        W = {name: B.weights(Q4_K, r, c, L, seed=101 + r + 7 * c, staging=staging) for name, r, c in LAYER}
        x0, _ = B.activation(D_, 1, 80, outliers=True)
        xo, _ = B.activation(D_, 1, 81, outliers=True)
        wn1, wn2 = B.buf(D_ * 4), B.buf(D_ * 4)
        flh.fill_normal(wn1, D_, 81, s, mean=1.0, std=0.1)
        flh.fill_normal(wn2, D_, 82, s, mean=1.0, std=0.1)
        xn1, _ = B.activation(D_, 1, 83, outliers=False)
        xn2, _ = B.activation(D_, 1, 84, outliers=False)
        h, _ = B.activation(F_, 1, 85, outliers=False)
        y = {name: B.buf(r * 4) for name, r, c in LAYER}
        gu = y["gate_up"]
        for i in range(launches):
            l = i % L
            flh.rmsnorm_stream_dot(Q4_K, W["qkv"][l], 6144, D_, x0, wn1, 1e-5, xn1, y["qkv"], s)
            flh.act_q8_stream_dot(Q4_K, W["o"][l], D_, D_, xo, y["o"], s)
            flh.rmsnorm_stream_dot(Q4_K, W["gate_up"][l], 2 * F_, D_, x0, wn2, 1e-5, xn2, gu, s)
            flh.silu_mul_act_q8(gu, gu.ptr + F_ * 4, h, F_, 1, 2 * F_, col_stride(flh, F_), s)
            flh.stream_dot(Q4_K, W["down"][l], D_, F_, h, y["down"], s)
    elif kind == "moe":
        E, K, D, F = 8, 2, 4096, 14336
        gu_b = 2 * F * flh.row_bytes(Q4_K, D)
        dn_b = D * flh.row_bytes(Q4_K, F)
        gu = B.weights(Q4_K, E * 2 * F, D, 1, seed=300, staging=staging)[0]
        dn = B.weights(Q4_K, E * D, F, 1, seed=400, staging=staging)[0]
        stD, stF = col_stride(flh, D), col_stride(flh, F)
        x, _ = B.activation(D, ntok, 60, outliers=False)
        lb = B.buf(ntok * E * 4)
        lb.upload(np.random.default_rng(2).standard_normal(ntok * E).astype(np.float32), s)
        ids, gates = B.buf(ntok * K * 4), B.buf(ntok * K * 4)
        ygu, ydn = B.buf(ntok * K * 2 * F * 4), B.buf(ntok * K * D * 4)
        h = B.buf(ntok * K * stF * 4)
        h.zero(s)
        yo = B.buf(ntok * D * 4)
        for _ in range(launches):
            flh.router_moe_dot(Q4_K, gu, gu_b, 2 * F, D, lb, ntok, E, K, 1, 1.0, ids, gates, x, stD,
                               False, ygu, 2 * F, s)
            flh.silu_mul_act_q8(ygu, ygu.ptr + F * 4, h, F, ntok * K, 2 * F, stF, s)
            flh.moe_dot(Q4_K, dn, dn_b, D, F, ids, ntok, K, E, h, stF, True, ydn, D, s)
            flh.wmerge(ydn, gates, None, None, yo, 1.0, K, D, 0, ntok, K * D, D, s)
    s.sync()
    for b in B.bufs:
        b.close()
    B.bufs.clear()


def traffic_from_profile():
    """HBM bytes per launch of the step's dominant kernel (the fused ACT_Q8 +
    gate/up launch), from the committed rocprofv3 --pmc summary
    (profiles/pmc_q4_K_gate_up_28672x4096_fused.json; FETCH_SIZE and
    WRITE_SIZE scaled by a 256 MiB copy's readings, profiles/q4_K_gate_up_28672x4096.md)."""
    f = os.path.join(ROOT, "profiles", "pmc_q4_K_gate_up_28672x4096_fused.json")
    try:
        with open(f) as fh:
            return json.load(fh).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def bench_moe(flh, B, s, staging, cpu_in):
    """Mixtral-style MoE FFN: router + grouped gate/up (one launch) -> silu*up +
    ACT_Q8 (one launch) -> grouped down -> weighted merge.  Three copies of the
    expert set rotate, so the routed experts of consecutive steps (198 MB per
    step at batch 1) cycle through more than 2x the 256 MB Infinity Cache."""
    E, K, D, F = 8, 2, 4096, 14336
    gu_b = 2 * F * flh.row_bytes(Q4_K, D)
    dn_b = D * flh.row_bytes(Q4_K, F)
    copies = 3
    gu = [B.weights(Q4_K, E * 2 * F, D, 1, seed=300 + c, staging=staging)[0] for c in range(copies)]
    dn = [B.weights(Q4_K, E * D, F, 1, seed=400 + c, staging=staging)[0] for c in range(copies)]
    out = {"ops": {}}
    rng = np.random.default_rng(2)
    for ntok in (1, 8):
        stD, stF = col_stride(flh, D), col_stride(flh, F)
        x, _ = B.activation(D, ntok, 60, outliers=False)
        logits = B.buf(ntok * E * 4)
        lg = [rng.standard_normal(ntok * E).astype(np.float32) for _ in range(copies)]
        ids = B.buf(ntok * K * 4)
        gates = B.buf(ntok * K * 4)
        ygu = B.buf(ntok * K * 2 * F * 4)
        h = B.buf(ntok * K * stF * 4)
        h.zero(s)
        ydn = B.buf(ntok * K * D * 4)
        yo = B.buf(ntok * D * 4)
        lbufs = []
        for c in range(copies):
            lb = B.buf(ntok * E * 4)
            lb.upload(lg[c], s)
            lbufs.append(lb)

        def issue(i):
            c = i % copies
            # router + grouped gate/up in one launch (same bits as router_sel, moe_dot)
            flh.router_moe_dot(Q4_K, gu[c], gu_b, 2 * F, D, lbufs[c], ntok, E, K, 1, 1.0, ids, gates, x, stD,
                               False, ygu, 2 * F, s)
            flh.silu_mul_act_q8(ygu, ygu.ptr + F * 4, h, F, ntok * K, 2 * F, stF, s)
            flh.moe_dot(Q4_K, dn[c], dn_b, D, F, ids, ntok, K, E, h, stF, True, ydn, D, s)
            flh.wmerge(ydn, gates, None, None, yo, 1.0, K, D, 0, ntok, K * D, D, s)

        us = B.time_graph(issue, 16)
        # bytes actually streamed: distinct experts per step
        distinct = []
        for c in range(copies):
            ll = lg[c].reshape(ntok, E)
            sel = set()
            for t in range(ntok):
                sel.update(np.argsort(-ll[t], kind="stable")[:K].tolist())
            distinct.append(len(sel))
        nb = int(np.mean(distinct) * (gu_b + dn_b))
        # CPU figure: the reference runs every (token, slot) pair's gate/up
        # and down dots on its own (src/model/decoder.cpp:941-996, no
        # grouping); the routed experts of copy 0, each token's x and each
        # pair's down input (a column with its appendices)
        hx = x.download(np.float32, ntok * stD, s)
        hh = h.download(np.float32, ntok * K * stF, s)
        wgu, wdn, cases = {}, {}, []
        for t in range(ntok):
            for e in np.argsort(-lg[0].reshape(ntok, E)[t], kind="stable")[:K].tolist():
                if e not in wgu:
                    wgu[e] = gu[0].download(np.uint8, gu_b, s, offset=e * gu_b)
                    wdn[e] = dn[0].download(np.uint8, dn_b, s, offset=e * dn_b)
                p = len(cases) // 2
                cases += [(Q4_K, wgu[e], 2 * F, D, hx[t * stD:(t + 1) * stD], stD, 1),
                          (Q4_K, wdn[e], D, F, hh[p * stF:(p + 1) * stF], stF, 1)]
        cpu_in[f"moe_q4_K_top2of8_batch{ntok}"] = cases
        out["ops"][f"moe_q4_K_top2of8_batch{ntok}"] = {
            "us": round(us, 3), "weight_bytes": nb, "distinct_experts": float(np.mean(distinct)),
            "GBs": round(nb / us / 1e3, 1), "pct_hbm": round(100 * nb / us / 1e3 / HBM_PEAK_GBS, 2)}
    return out


def host_case(flh, s, fmt, w, rows, cols, x, st, nx):
    """Host copy of one matvec's bytes (weights, activation columns with their
    appendices) for the CPU baseline."""
    return [(fmt, w.download(np.uint8, rows * flh.row_bytes(fmt, cols), s), rows, cols,
             x.download(np.float32, nx * st, s), st, nx)]


def cpu_share():
    """Host cores this process may use: its affinity set, capped by the
    thread share the box gives it (OMP_NUM_THREADS)."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(cap)) if cap.isdigit() and int(cap) > 0 else n


def cpu_model():
    """/proc/cpuinfo's model name with its family / model / stepping numbers
    (a virtualised host may report only a short name)."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = line.split(":", 1)
                info.setdefault(k.strip(), v.strip())
            elif info:
                break
    except OSError:
        return ""
    return (f"{info.get('model name', '')} (family {info.get('cpu family', '?')}, model "
            f"{info.get('model', '?')}, stepping {info.get('stepping', '?')})")


def cpu_baseline(flh, s, W, xin, cpu_in):
    """The reference CPU quantized-dot path (exec_task_cpu, int8 dots with the
    CPU default masks) on the host cores: rows split over T threads as
    tools/membench.cu:276-300 does.  value: the headline layer step (4 Q4_K
    matvecs on the same bytes and appendices); configs: every other
    BASELINE config on its own bytes.  Each figure repeats its work for about
    1.5 s (the single-thread layer figure about 3 s)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Oracle, REF_SO
    kind = "reference" if os.path.exists(REF_SO) else "port"
    orc = Oracle(ref=(kind == "reference"))
    T = cpu_share()
    layer = []
    for name, r, c in LAYER:
        x, st = xin[name]
        layer += host_case(flh, s, Q4_K, W[name][0], r, c, x, st, 1)

    def run(cases, threads):
        for fmt, w, r, c, xb, st, nx in cases:
            y = np.zeros(nx * r, dtype=np.float32)
            orc.stream_dot(fmt, w, r, c, xb, y, nx=nx, xstride=st, ystride=r, fast=True, threads=threads)

    def rate(cases, threads, secs):
        nbytes = sum(w.size for _, w, _, _, _, _, _ in cases)
        run(cases, threads)
        reps, t0 = 0, time.perf_counter()
        while True:
            run(cases, threads)
            reps += 1
            el = time.perf_counter() - t0
            if el > secs:
                break
        return nbytes, reps, el

    for case, (name, r, c) in zip(layer, LAYER):
        cpu_in[f"q4_K_{name}_{r}x{c}"] = [case]
    nb, reps, el = rate(layer, T, 1.5)
    val = nb * reps / el / 1e9
    nb1, reps1, el1 = rate(layer, 1, 3.0)
    configs = {}
    for name, cases in cpu_in.items():
        cb, cr, ce = rate(cases, T, 1.5)
        configs[name] = {"us": round(ce / cr * 1e6, 1), "GBs": round(cb * cr / ce / 1e9, 3),
                         "weight_bytes": cb, "reps": cr}
    return {"value": round(val, 3), "unit": "GB/s", "cores": T, "kind": kind,
            "us_per_step": round(el / reps * 1e6, 1), "value_1thread": round(nb1 * reps1 / el1 / 1e9, 3),
            "cpu": cpu_model(), "configs": configs,
            "sample": f"layer step (4 Q4_K matvecs, {nb} weight bytes) repeated {reps} times in "
                      f"{el:.2f} s on {T} threads (and {reps1} times in {el1:.2f} s on 1 thread); each "
                      f"other config repeated for ~1.5 s on {T} threads (configs.*.reps); reference "
                      f"exec_task_cpu int8 path (fast, CPU default masks), rows split over threads"}


if __name__ == "__main__":
    main()
