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

}  // extern "C"
