// ref_shim.cpp -- extern "C" entry points over the reference's own CPU code,
// compiled from /root/reference sources in place (oracle/Makefile, target
// `ref`) into oracle/_ref/libflref.so.  TEST INFRASTRUCTURE ONLY: used by
// tests/golden/make_golden.py (in this container) to write golden vectors
// and to cross-check oracle/fl_oracle.c.  Nothing here is product code, and
// no reference source is copied: the reference headers are included from
// the read-only tree by -I.
#include "fastllm/fastllm.h"
#include "runtime/quants.h"
#include "runtime/kernels.h"
#include "runtime/decode_params.h"
#include <cstring>
#include <thread>
#include <vector>

using namespace fastllm;

extern "C" {

float ref_half2float(uint16_t h) { return fl_half2float(h); }
uint16_t ref_float2half(float f) { return fl_float2half(f); }

// src/runtime/kernels.h:162 dequant_chunk over whole rows
void ref_dequant_rows(int fmt, const uint8_t * w, uint32_t rows, uint32_t cols,
                      float * out) {
    const uint64_t rb = fl_row_bytes((Fmt)fmt, cols);
    for (uint32_t r = 0; r < rows; ++r)
        dequant_chunk((Fmt)fmt, w + r * rb, 0, cols, out + (size_t)r * cols);
}

// src/runtime/quants.h:404 fl_exec_act_q8 on one column buffer
void ref_act_q8(float * x, uint32_t cols) {
    Task t{};
    t.kind = TaskKind::ACT_Q8;
    t.x = x;
    t.y = (void *)fl_xq_of(x, cols);
    t.rows = cols / 32;
    t.cols = cols;
    fl_exec_act_q8(t);
}

size_t ref_x_alloc_bytes(uint32_t cols) { return fl_x_alloc_bytes(cols); }

// src/runtime/kernels.h:1002 exec_task_cpu, one STREAM_DOT (or _IDX) tile
void ref_stream_dot(int fmt, const void * w, uint32_t rows, uint32_t cols,
                    const float * x, float * y, uint32_t nx, uint32_t xstride,
                    uint32_t ystride, int fast, uint32_t i8_mask,
                    uint32_t i8k_mask, const uint32_t * id_slot,
                    uint64_t estride) {
    Task t{};
    t.kind = id_slot ? TaskKind::STREAM_DOT_IDX : TaskKind::STREAM_DOT;
    t.fmt = (Fmt)fmt;
    t.w = w;
    t.rows = rows;
    t.cols = cols;
    t.w_bytes = (uint64_t)rows * fl_row_bytes((Fmt)fmt, cols);
    t.x = x;
    t.y = y;
    t.nx = nx;
    t.xstride = xstride;
    t.ystride = ystride;
    t.aux = id_slot;
    t.aux2 = estride;
    exec_task_cpu(t, fast != 0, i8_mask, i8k_mask);
}

// rows split across nthreads std::threads, the CPU probe harness of
// tools/membench.cu:276-300 (one exec_task_cpu per row range)
void ref_stream_dot_mt(int fmt, const void * w, uint32_t rows, uint32_t cols,
                       const float * x, float * y, uint32_t nx, uint32_t xstride,
                       uint32_t ystride, int fast, uint32_t i8_mask,
                       uint32_t i8k_mask, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    const uint64_t rb = fl_row_bytes((Fmt)fmt, cols);
    std::vector<std::thread> th;
    for (int t = 0; t < nthreads; ++t) {
        const uint32_t r0 = (uint32_t)((uint64_t)rows * t / nthreads);
        const uint32_t r1 = (uint32_t)((uint64_t)rows * (t + 1) / nthreads);
        th.emplace_back([=] {
            ref_stream_dot(fmt, (const uint8_t *)w + r0 * rb, r1 - r0, cols, x, y + r0, nx,
                           xstride, ystride, fast, i8_mask, i8k_mask, nullptr, 0);
        });
    }
    for (auto & t : th) t.join();
}

// canonical serial path (src/runtime/runtime_internal.h:240-257)
void ref_stream_dot_canonical(int fmt, const void * w, uint32_t rows,
                              uint32_t cols, const float * x, float * y,
                              uint32_t nx, uint32_t xstride, uint32_t ystride) {
    Task t{};
    t.kind = TaskKind::STREAM_DOT;
    t.fmt = (Fmt)fmt;
    t.w = w; t.rows = rows; t.cols = cols;
    t.w_bytes = (uint64_t)rows * fl_row_bytes((Fmt)fmt, cols);
    t.x = x; t.y = y; t.nx = nx; t.xstride = xstride; t.ystride = ystride;
    exec_task_scalar_host(t);
}

// the reference's IQ codebooks and sign table (src/model/iq_tables.h), for
// hashing: fixtures record only a digest of them, never the values
void ref_iq_tables(uint64_t * g2, uint32_t * g3, uint8_t * signs) {
    for (int i = 0; i < 256; ++i) { g2[i] = fl_kIq2xxsGrid(i); g3[i] = fl_kIq3xxsGrid(i); }
    for (int i = 0; i < 128; ++i) signs[i] = fl_kIqSigns(i);
}

void ref_router_sel(const float * logits, uint32_t n_expert, uint32_t top_k,
                    uint32_t norm, float scale, uint32_t * ids, float * gates) {
    RouterP p{logits, ids, gates, n_expert, top_k, norm, scale};
    fl_op_router_sel(p);
}
void ref_rmsnorm(const float * wnorm, const float * x, float * y, float eps, uint32_t n) {
    RmsNormP p{wnorm, x, y, eps, n};
    fl_op_rmsnorm(p);
}
void ref_silu_mul(const float * gate, const float * up, float * h, uint32_t n) {
    SiluMulP p{gate, up, h, n};
    fl_op_silu_mul(p);
}
void ref_wmerge(const float * parts, const float * gates, const float * add1,
                const float * add2, float * y, float scale, uint32_t n_parts,
                uint32_t n, uint32_t n_full) {
    WmergeP p{parts, gates, add1, add2, y, scale, n_parts, n, n_full};
    fl_op_wmerge(p);
}


// A frozen MoE FFN graph of one token, built with the reference's own Arena
// and Graph (include/fastllm/fastllm.h:103-124) in the shape the decoder
// emits (src/model/decoder.cpp:941-996) and run by run_serial
// (src/runtime/graph.cpp:116-148, the canonical exec_task_scalar path):
//   0 ACT_Q8(x)  1 ROUTER_SEL(logits)
//   per slot k: gate/up STREAM_DOT_IDX in two row tiles, SILU_MUL, ACT_Q8(h),
//               down STREAM_DOT_IDX into parts[k]
//   WMERGE(parts, gates, add1 = x) -> y, SIGNAL
// x: d floats, logits: ne floats, wgu: ne experts of 2*ff Q4_K rows of d
// columns, wdn: ne experts of d Q6_K rows of ff columns.  Copies the arena
// region (task table first) before and after the run into pre / post
// (cap bytes each) and reports the region size, the task count and the
// offsets of the named buffers:
//   off[0] x  off[1] logits  off[2] ids  off[3] gates  off[4] wgu  off[5] wdn
//   off[6] gu (topk * 2ff floats)  off[7] h (topk columns, hstride floats)
//   off[8] parts (topk * d)  off[9] y (d)  off[10] router P  off[11] silu P
//   (topk)  off[12] wmerge P  off[13] hstride (floats, a value)
// Returns 0, or -1 if cap is too small.
int ref_run_serial_moe(uint32_t d, uint32_t ff, uint32_t ne, uint32_t topk, const float * x,
                       const float * logits, const uint8_t * wgu, const uint8_t * wdn,
                       uint8_t * pre, uint8_t * post, size_t cap, uint64_t * used_out,
                       uint32_t * ntask_out, uint64_t * off) {
    const uint64_t rb4 = fl_row_bytes(Fmt::Q4_K, d), rb6 = fl_row_bytes(Fmt::Q6_K, ff);
    auto arena = Arena::create(64u << 20);
    auto g = Graph::create(*arena, 64);
    uint8_t * base = (uint8_t *)g->tasks();
    auto A = [&](size_t n) { return (uint8_t *)arena->alloc(n, 128); };
    const size_t xb = fl_x_alloc_bytes(d), hb = (fl_x_alloc_bytes(ff) + 127) & ~(size_t)127;
    uint8_t * X = A(xb);
    float * LG = (float *)A(ne * 4);
    uint32_t * IDS = (uint32_t *)A(topk * 4);
    float * GT = (float *)A(topk * 4);
    uint8_t * WGU = A((size_t)ne * 2 * ff * rb4);
    uint8_t * WDN = A((size_t)ne * d * rb6);
    float * GU = (float *)A((size_t)topk * 2 * ff * 4);
    uint8_t * H = A(hb * topk);
    float * PARTS = (float *)A((size_t)topk * d * 4);
    float * Y = (float *)A(d * 4);
    RouterP * rp = (RouterP *)A(sizeof(RouterP));
    SiluMulP * sp = (SiluMulP *)A(sizeof(SiluMulP) * topk);
    WmergeP * wp = (WmergeP *)A(sizeof(WmergeP));
    memcpy(X, x, d * 4);
    memcpy(LG, logits, ne * 4);
    memcpy(WGU, wgu, (size_t)ne * 2 * ff * rb4);
    memcpy(WDN, wdn, (size_t)ne * d * rb6);
    *rp = RouterP{LG, IDS, GT, ne, topk, 1u, 1.0f};
    auto act = [&](uint8_t * col, uint32_t cols) {
        Task t{};
        t.kind = TaskKind::ACT_Q8;
        t.x = col;
        t.y = (void *)fl_xq_of((float *)col, cols);
        t.rows = cols / 32;
        t.cols = cols;
        return g->add(t);
    };
    auto dot = [&](Fmt f, const uint8_t * w, uint32_t rows, uint32_t cols, const void * xx, float * y,
                   const uint32_t * slot, uint64_t estride) {
        Task t{};
        t.kind = TaskKind::STREAM_DOT_IDX;
        t.fmt = f;
        t.w = w;
        t.w_bytes = (uint64_t)rows * fl_row_bytes(f, cols);
        t.x = xx;
        t.y = y;
        t.rows = rows;
        t.cols = cols;
        t.aux = slot;
        t.aux2 = estride;
        return g->add(t);
    };
    const uint32_t t_act = act(X, d);
    Task tr{};
    tr.kind = TaskKind::ROUTER_SEL;
    tr.aux = rp;
    const uint32_t t_rt = g->add(tr);
    std::vector<uint32_t> downs;
    for (uint32_t k = 0; k < topk; ++k) {
        const uint32_t ta = dot(Fmt::Q4_K, WGU, ff, d, X, GU + (size_t)k * 2 * ff, IDS + k, 2 * ff * rb4);
        const uint32_t tb = dot(Fmt::Q4_K, WGU + ff * rb4, ff, d, X, GU + (size_t)k * 2 * ff + ff, IDS + k,
                                2 * ff * rb4);
        float * h = (float *)(H + hb * k);
        sp[k] = SiluMulP{GU + (size_t)k * 2 * ff, GU + (size_t)k * 2 * ff + ff, h, ff};
        Task ts{};
        ts.kind = TaskKind::SILU_MUL;
        ts.aux = &sp[k];
        const uint32_t tsl = g->add(ts);
        const uint32_t tq = act((uint8_t *)h, ff);
        const uint32_t td = dot(Fmt::Q6_K, WDN, d, ff, h, PARTS + (size_t)k * d, IDS + k, (uint64_t)d * rb6);
        g->edge(t_act, ta); g->edge(t_act, tb);
        g->edge(t_rt, ta); g->edge(t_rt, tb);
        g->edge(ta, tsl); g->edge(tb, tsl);
        g->edge(tsl, tq); g->edge(tq, td);
        downs.push_back(td);
    }
    *wp = WmergeP{PARTS, GT, (const float *)X, nullptr, Y, 1.0f, topk, d, 0u};
    Task tw{};
    tw.kind = TaskKind::WMERGE;
    tw.aux = wp;
    const uint32_t t_wm = g->add(tw);
    for (uint32_t td : downs) g->edge(td, t_wm);
    g->edge(t_rt, t_wm);
    Task tsg{};
    tsg.kind = TaskKind::SIGNAL;
    const uint32_t t_sig = g->add(tsg);
    g->edge(t_wm, t_sig);
    g->freeze();
    const size_t used = arena->used();
    if (used > cap) return -1;
    memcpy(pre, base, used);
    run_serial(*g);
    memcpy(post, base, used);
    *used_out = used;
    *ntask_out = g->size();
    const uint8_t * ptrs[13] = {X, (uint8_t *)LG, (uint8_t *)IDS, (uint8_t *)GT, WGU, WDN, (uint8_t *)GU, H,
                                (uint8_t *)PARTS, (uint8_t *)Y, (uint8_t *)rp, (uint8_t *)sp, (uint8_t *)wp};
    for (int i = 0; i < 13; ++i) off[i] = (uint64_t)(ptrs[i] - base);
    off[13] = hb / 4;
    return 0;
}

}  // extern "C"
