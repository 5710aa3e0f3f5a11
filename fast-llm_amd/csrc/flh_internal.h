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

// RMSNORM in front of a fused ACT_Q8 dot: the activation buffer of the dot
// (DotArgs::x) receives y = (x * s) * wn and its appendices, with
// s = 1 / sqrtf(sum(x^2) / n + eps) over the column x (fl_op_rmsnorm,
// src/runtime/decode_params.h:101-106).
struct NormArgs {
    const float * x;
    const float * wn;
    float eps;
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
    // fused ROUTER_SEL (rt_logits not null; n_expert <= 64, top_k <= 8,
    // ntok * top_k <= 256): every workgroup routes the tokens itself, and
    // workgroup (0, 0) also writes ids (the ids field) and rt_gates
    const float * rt_logits = nullptr;
    uint32_t rt_norm = 0;
    float rt_scale = 1.f;
    float * rt_gates = nullptr;
};

int num_cus();

// grid rows of a grouped expert matvec: the experts that can be active
inline uint32_t moe_rows(const MoeArgs & a) {
    const uint32_t pairs = a.ntok * a.top_k;
    return pairs < a.n_expert ? pairs : a.n_expert;
}

// Each returns hipSuccess-style 0 or a negative flh error code.
int launch_act_q8(float * x, void * y_q81, uint32_t cols, uint32_t nx,
                  uint32_t xstride, hipStream_t s);
// RMSNORM of one column, with the ACT_Q8 of its output when app
int launch_rmsnorm_act_q8(const float * x, const float * wnorm, float * y, uint32_t n, float eps, bool app,
                          hipStream_t s);
// SILU_MUL over ncol columns followed by ACT_Q8 of h, in one launch
int launch_silu_act_q8(const float * gate, const float * up, float * h, uint32_t n, uint32_t ncol,
                       uint32_t gstride, uint32_t hstride, hipStream_t s);
int launch_dot_i8k(int fmt, const DotArgs & a, hipStream_t s);    // Q4_K, Q6_K x q8_K
// LDS-staged variant; FLH_ERR_UNSUPPORTED (nothing launched) if the shape
// does not fit its plan
// Launch tuning.  The defaults are the measured-best settings; flh_init()
// (every call) re-reads the development overrides from the environment, so a
// launch never reads the environment itself.
struct Tune {
    uint32_t fuse_max_cols = 8192;      // FLH_FUSE_MAX_COLS: widest activation fused into its dot
    // streaming kernel, FLH_KS_TUNE = "wgs_per_cu,nr,D[,pro]" (0 = default)
    uint32_t ks_wgs_per_cu = 0, ks_nr = 0, ks_D = 0, ks_pro = 0;
    // single-column 8-wave workgroups, FLH_KS_W8 = "mode,wgs_per_cu" (mode bits
    // 1: fused, > 16 superblocks; 2: fused, <= 16; 4: unfused, > 16; 8: unfused, <= 16)
    uint32_t ks_w8_mode = 7, ks_w8_wgs = 2;
    // register kernel, FLH_KQ_TUNE = "wgs_per_cu,nr,D"
    uint32_t kq_wgs_per_cu = 4, kq_nr = 0, kq_D = 2;
    // matrix-core kernel
    uint32_t mf_pro = 0;                // FLH_MFMA_PRO: chunks per wave before staging (0: the ring)
    uint32_t mf_D = 0, mf_nrb = 0;      // FLH_MFMA_TUNE = "D,nrb[,kh]" (0: planned)
    int mf_kh = -1;                     //   kh: 1 force K halves, 0 never, -1 planned
    bool mf_xc = true;                  // FLH_MFMA_XC=0: no activations-in-chunk mode
    bool mf_own = true;                 // FLH_MFMA_OWN=0: parked terms and a fold pass, not register sums
    uint32_t mf_min_cols = 0;           // FLH_MFMA_MIN_COLS (0: 2 above 4096 columns, else 3)
    bool no_mfma = false;               // FLH_NO_MFMA=1: never the matrix-core kernels
    bool no_q6mf = false;               // FLH_NO_Q6MF=1: several Q6_K columns off the matrix cores
    uint32_t q6mf_rows = 12288, q6mf_cols = 5;  // FLH_Q6MF_MIN = "rows,cols": the smallest shape sent there
    // superblock-per-lane single-column kernel, FLH_SBL = "on,waves,wgs_per_cu,max_wgs,pre"
    // (0 = default; max_wgs caps the grid, for tests of long per-wave chunk
    // lists; pre = waves requesting a chunk before the activation lands, 0: half, 255: all)
    uint32_t sbl = 1, sbl_w = 0, sbl_wpc = 0, sbl_gmax = 0, sbl_pre = 0;
    uint32_t sbl_nx_dep = 0;            // FLH_SBL_NX_DEP: ring stages of the several-column kernel (0: planned)
    uint32_t gguf_threads = 0;          // FLH_GGUF_THREADS: host copy threads of an upload (0: all, <= 16)
};
const Tune & tune();
void load_tune();

int launch_dot_kstream(int fmt, const DotArgs & a, hipStream_t s);
// One column, one superblock (K formats) or four 32-weight blocks per lane
// (flh_dot_sbl.hip): Q4_K (fuse: ACT_Q8 of the fp32 column in the same
// launch), Q6_K, Q8_0, Q5_0, IQ2_XXS, IQ3_XXS.  FLH_ERR_UNSUPPORTED (nothing
// launched) if the shape does not fit its plan or another kernel is faster.
int launch_dot_sbl(int fmt, const DotArgs & a, bool fuse, hipStream_t s, const NormArgs * norm = nullptr);
// 2..8 activation columns of Q8_0 / Q5_0 / IQ2_XXS / IQ3_XXS on the
// superblock-per-lane layout (FLH_ERR_UNSUPPORTED: nothing launched)
int launch_dot_sbl_nx(int fmt, const DotArgs & a, hipStream_t s);
// RMSNORM -> ACT_Q8 -> Q4_K one-column dot on the four-lanes-per-superblock
// kernel (FLH_ERR_UNSUPPORTED: nothing launched)
int launch_norm_dot_kstream(const DotArgs & a, const NormArgs & nm, hipStream_t s);
// largest dynamic LDS of one workgroup on the current device
size_t lds_limit();
// a kernel's static LDS, and whether a launch of it with dyn bytes of dynamic
// LDS fits one workgroup (FLH_ERR_UNSUPPORTED with the message otherwise)
size_t static_lds(const void * kern);
int lds_fits(const void * kern, size_t dyn, const char * what);
// ACT_Q8 fused into the kstream dot: quantises x (fp32) in-kernel, writes both
// appendices (workgroup 0), then streams; same bytes and results as
// launch_act_q8 followed by launch_dot_kstream
int launch_act_dot_kstream(int fmt, const DotArgs & a, hipStream_t s);
// Q4_K x q8_K, 1..16 columns, on the int8 matrix cores (flh_dot_mfma.hip);
// FLH_ERR_UNSUPPORTED (nothing launched) if the shape does not fit its plan
int launch_dot_mfma(int fmt, const DotArgs & a, hipStream_t s);
// grouped expert variant (MoE, Q4_K, batches of several tokens)
int launch_moe_mfma(int fmt, const MoeArgs & a, hipStream_t s);
// fewest columns for which STREAM_DOT uses launch_dot_mfma
uint32_t mfma_min_cols(uint32_t cols);
int mfma_plan(uint32_t rows, uint32_t cols, uint32_t nx, uint32_t * out);
int launch_dot_i8_q8_0(const DotArgs & a, hipStream_t s);         // Q8_0 x q8_1
int launch_dot_i8_q5_0(const DotArgs & a, hipStream_t s);         // Q5_0 x q8_1
int launch_dot_i8_k(int fmt, const DotArgs & a, hipStream_t s);   // Q4_K, Q6_K x q8_1
int launch_dot_i8_iq(int fmt, const DotArgs & a, hipStream_t s);  // IQ2_XXS, IQ3_XXS x q8_1
int launch_dot_canonical(int fmt, const DotArgs & a, hipStream_t s);
int launch_dot_fast_f32(int fmt, const DotArgs & a, hipStream_t s);
int launch_dequant(int fmt, const uint8_t * w, uint32_t rows, uint32_t cols,
                   float * out, hipStream_t s);
int launch_moe_i8k(int fmt, const MoeArgs & a, hipStream_t s);
int launch_dot_q6mf(const DotArgs & a, hipStream_t s);
// LDS-staged grouped expert kernel; FLH_ERR_UNSUPPORTED if it does not fit
int launch_moe_kstream(int fmt, const MoeArgs & a, hipStream_t s);
int launch_moe_sbl(int fmt, const MoeArgs & a, hipStream_t s);
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

}  // namespace flh
