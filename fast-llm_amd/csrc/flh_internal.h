// flh_internal.h -- launcher interface between the C-ABI layer (flh_api.cpp)
// and the kernel translation units.  Not installed; include/fastllm_hip.h is
// the public boundary.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace flh {

// One STREAM_DOT launch: y[p*ystride + r] += dot(W[r], x + p*xstride),
// r < rows, p < nx.  W = w (+ *id_slot * estride when id_slot != nullptr,
// resolved on the device: the id is written by an earlier kernel).
struct DotArgs {
    const uint8_t * w;
    const uint32_t * id_slot;
    uint64_t estride;
    const float * x;
    float * y;
    uint32_t rows, cols, nx, xstride, ystride;
};

// Grouped expert launch (MoE): for every expert e with at least one routed
// (token, slot) pair, the columns are those pairs:
//   y[(tok*top_k + slot)*ystride + r] += dot(W_e[r], x + xcol(tok,slot)*xstride)
// where xcol = tok when x_per_slot == 0 (shared hidden state per token) and
// tok*top_k + slot otherwise (per-slot activations, e.g. the down input).
struct MoeArgs {
    const uint8_t * w;        // expert 0 base
    uint64_t estride;         // bytes between experts
    const uint32_t * ids;     // [ntok * top_k] expert ids
    const float * x;
    float * y;
    uint32_t rows, cols, ntok, top_k, n_expert, xstride, ystride, x_per_slot;
};

int num_cus();

// Each returns hipSuccess-style 0 or a negative flh error code.
int launch_act_q8(float * x, void * y_q81, uint32_t cols, uint32_t nx,
                  uint32_t xstride, hipStream_t s);
int launch_dot_i8k(int fmt, const DotArgs & a, hipStream_t s);    // Q4_K, Q6_K x q8_K
// LDS-staged variant; FLH_ERR_UNSUPPORTED (nothing launched) if the shape
// does not fit its plan
int launch_dot_kstream(int fmt, const DotArgs & a, hipStream_t s);
// ACT_Q8 fused into the kstream dot: quantises x (fp32) in-kernel, writes both
// appendices (workgroup 0), then streams; same bytes and results as
// launch_act_q8 followed by launch_dot_kstream
int launch_act_dot_kstream(int fmt, const DotArgs & a, hipStream_t s);
int launch_dot_i8_q8_0(const DotArgs & a, hipStream_t s);         // Q8_0 x q8_1
int launch_dot_i8_k(int fmt, const DotArgs & a, hipStream_t s);   // Q4_K, Q6_K x q8_1
int launch_dot_canonical(int fmt, const DotArgs & a, hipStream_t s);
int launch_dot_fast_f32(int fmt, const DotArgs & a, hipStream_t s);
int launch_dequant(int fmt, const uint8_t * w, uint32_t rows, uint32_t cols,
                   float * out, hipStream_t s);
int launch_moe_i8k(int fmt, const MoeArgs & a, hipStream_t s);
// LDS-staged grouped expert kernel; FLH_ERR_UNSUPPORTED if it does not fit
int launch_moe_kstream(int fmt, const MoeArgs & a, hipStream_t s);
int launch_router_sel(const float * logits, uint32_t ntok, uint32_t n_expert,
                      uint32_t top_k, uint32_t norm, float scale,
                      uint32_t * ids, float * gates, hipStream_t s);
int launch_silu_mul(const float * gate, const float * up, float * h, uint32_t n,
                    uint32_t ncol, uint32_t gstride, uint32_t hstride, hipStream_t s);
int launch_wmerge(const float * parts, const float * gates, const float * add1,
                  const float * add2, float * y, float scale, uint32_t n_parts,
                  uint32_t n, uint32_t n_full, uint32_t ncol, uint32_t pstride,
                  uint32_t ystride, hipStream_t s);
int launch_merge(const float * x, float * y, uint32_t rows, uint32_t nparts,
                 hipStream_t s);
int launch_quantize_weights(int fmt, const float * src, uint32_t rows,
                            uint32_t cols, uint8_t * dst, hipStream_t s);
int launch_fill_normal(float * dst, size_t n, uint64_t seed, float mean,
                       float stddev, float outlier_frac, float outlier_scale,
                       hipStream_t s);

// ------------------------------------------------------------------ plans --
// A frozen task table compiled into ops for the persistent plan executor
// (flh_plan.hip).  Op k's work is split into nitems items with global
// indices [item0, item0 + nitems); items are dealt to the resident
// workgroups round-robin in index order, and an item starts its activation
// reads only when every producer op (bitmask prod) has completed all items.
constexpr int PLAN_MAX_OPS = 32;
enum : uint32_t { PLOP_DOT = 0, PLOP_ACT = 1 };
enum : uint32_t { PLF_FUSE = 1, PLF_XREG = 2, PLF_SILU = 4, PLF_NOQ = 8 };
struct PlanOp {
    const uint8_t * w;     // DOT: weights (16-byte aligned)
    const float * x;       // DOT: activation column; ACT: input (SILU: gate)
    float * y;             // DOT: output (+=); ACT: column quantised in place (SILU: h)
    const float * u;       // ACT with SILU: up operand
    uint32_t kind, flags;
    uint32_t rows, cols;   // DOT: matrix shape; ACT: cols = elements
    uint32_t nr;           // DOT: rows per item; ACT: 256-element chunks per item (4)
    uint32_t item0, nitems;
    uint32_t prod;         // producer ops
};
struct PlanArgs {
    const PlanOp * ops;    // device copy, sorted by item0
    uint32_t * ctl;        // [0] finished workgroups, [1] error flag, [2 + k] items done of op k
    const uint8_t * wdummy;  // a valid weight address (re-read, unused, once a cursor is exhausted)
    uint64_t * trace;        // per-item timestamps (diagnostic builds only; null otherwise)
    uint32_t nops, nitems, spin_limit, term_off;
};
// the LDS plan of a plan launch
size_t plan_stage_bytes(int fmt);
int launch_plan(int fmt, const PlanArgs & a, uint32_t grid, size_t smb, hipStream_t s);
int plan_occupancy(int fmt, size_t smb, int * blocks_per_cu);

}  // namespace flh
