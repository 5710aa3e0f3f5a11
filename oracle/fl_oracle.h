/*
 * fl_oracle.h -- CPU restatement of the reference's quantized dot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * product path: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product (fast-llm_amd/) never links,
 * loads or falls back to it.
 *
 * Every function restates one function of the reference (qdox-labs/fast-llm)
 * and cites it as path:line.  Compiled with -ffp-contract=off, exactly like
 * the reference (CMakeLists.txt:13), so every float expression rounds once
 * per operation in source order.
 *
 * Parity pinning (how each function is checked, tests/test_oracle_*.py):
 *   - half2float: exhaustive over all 65536 halves against numpy float16.
 *   - float2half: reference KATs (tests/test_runtime.cpp:540-544) + numpy
 *     RNE sweep.
 *   - q4k_scale_min, dequant: closed-form per-element transcription
 *     (tests/test_quants.cpp:36-80 style) + golden vectors from oracle/_ref.
 *   - act quantizers: bsums == per-16 sums, one-step reconstruction,
 *     golden vectors from oracle/_ref (bit patterns of d, s, qs, bsums).
 *   - int8 dots: integer parts brute-forced on tiny inputs, full float
 *     bit patterns against oracle/_ref golden vectors, error budget vs f64.
 *   - router/silu/wmerge: reference KAT (tests/test_decode_ops.cpp:84-102)
 *     + oracle/_ref golden vectors.
 */
#ifndef FL_ORACLE_H
#define FL_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Fmt numeric values: include/fastllm/fastllm.h:56-57 */
enum { ORC_F32 = 0, ORC_Q8_0 = 1, ORC_Q5_0 = 2, ORC_Q4_K = 3, ORC_Q6_K = 4,
       ORC_IQ2_XXS = 5, ORC_IQ3_XXS = 6 };

float    orc_half2float(uint16_t h);
uint16_t orc_float2half(float f);
uint32_t orc_blk_elems(int fmt);
uint32_t orc_blk_bytes(int fmt);
uint64_t orc_row_bytes(int fmt, uint32_t cols);
void     orc_q4k_scale_min(int j, const uint8_t * s, uint8_t * d, uint8_t * m);

/* activation appendix layout (src/runtime/quants.h:302-330) */
size_t   orc_xq_offset(uint32_t cols);
size_t   orc_xqk_offset(uint32_t cols);
size_t   orc_x_alloc_bytes(uint32_t cols);

void orc_dequant_chunk(int fmt, const uint8_t * row, uint32_t elem0,
                       uint32_t n, float * out);
void orc_dequant_rows(int fmt, const uint8_t * w, uint32_t rows,
                      uint32_t cols, float * out);

float orc_dot_row(int fmt, const uint8_t * row, const float * x, uint32_t cols);
float orc_dot_row_fast(const float * row, const float * x, uint32_t cols);
float orc_dot_row_fast_q8_0(const uint8_t * row, const float * x, uint32_t cols);
float orc_dot_row_fast_dequant(int fmt, const uint8_t * row, const float * x,
                               uint32_t cols);

void orc_quantize_q8_1_block(const float * x, uint8_t * o36);
void orc_quantize_q8_K_block(const float * x, uint8_t * o292);
/* ACT_Q8 on one column: x is the base of an fl_x_alloc_bytes(cols) buffer */
void orc_act_q8(float * x, uint32_t cols);

float orc_dot_i8_q8_0(const uint8_t * row, const uint8_t * xq, uint32_t cols);
float orc_dot_i8_q5_0(const uint8_t * row, const uint8_t * xq, uint32_t cols);
float orc_dot_i8_q4_K(const uint8_t * row, const uint8_t * xq, uint32_t cols);
float orc_dot_i8_q6_K(const uint8_t * row, const uint8_t * xq, uint32_t cols);
/* IQ formats: codebook accessors, the sign-byte widening, the q8_1 dot */
uint64_t orc_iq2_grid(int i);
uint32_t orc_iq3_grid(int i);
uint8_t  orc_iq_signs(uint32_t s7);
float orc_dot_i8_iq(int fmt, const uint8_t * row, const uint8_t * xq, uint32_t cols);
float orc_dot_i8k_q4_K(const uint8_t * row, const uint8_t * xk, uint32_t cols);
float orc_dot_i8k_q6_K(const uint8_t * row, const uint8_t * xk, uint32_t cols);

/* exec_task_cpu STREAM_DOT semantics (src/runtime/kernels.h:1002-1258, x86
 * branches): y[p*ystride + r] += dot(W[r], x + p*xstride) for p < nx. */
void orc_stream_dot(int fmt, const uint8_t * w, uint32_t rows, uint32_t cols,
                    const float * x, float * y, uint32_t nx, uint32_t xstride,
                    uint32_t ystride, int fast, uint32_t i8_mask,
                    uint32_t i8k_mask);
/* same, rows split across nthreads std::thread-style workers (pthreads),
 * the CPU-baseline harness of tools/membench.cu:276-300 */
void orc_stream_dot_mt(int fmt, const uint8_t * w, uint32_t rows, uint32_t cols,
                       const float * x, float * y, uint32_t nx, uint32_t xstride,
                       uint32_t ystride, int fast, uint32_t i8_mask,
                       uint32_t i8k_mask, int nthreads);

/* MoE glue (src/runtime/decode_params.h:234-295) */
void orc_router_sel(const float * logits, uint32_t n_expert, uint32_t top_k,
                    uint32_t norm, float scale, uint32_t * ids, float * gates);
void orc_silu_mul(const float * gate, const float * up, float * h, uint32_t n);
void orc_rmsnorm(const float * wnorm, const float * x, float * y, float eps, uint32_t n);
void orc_wmerge(const float * parts, const float * gates, const float * add1,
                const float * add2, float * y, float scale, uint32_t n_parts,
                uint32_t n, uint32_t n_full);

#ifdef __cplusplus
}
#endif
#endif
