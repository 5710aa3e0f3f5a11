// flh_api.cpp -- the C-ABI boundary (include/fastllm_hip.h): device setup,
// device arena, streams/events, argument validation mirroring the
// reference's Graph::freeze() rules, per-task dispatch and row-tile fusion.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <stdlib.h>
#include <string>
#include <atomic>
#include <mutex>
#include "../../include/fastllm_hip.h"
#include "flh_common.h"
#include "flh_internal.h"
#include "flh_status.h"

namespace flh {

static thread_local std::string g_err;
static int g_device = -1;
static int g_cus = 256;

int set_error(int code, const char * msg) {
    g_err = msg ? msg : "";
    return code;
}
int hip_check(hipError_t e, const char * what) {
    if (e == hipSuccess) return FLH_OK;
    g_err = std::string(what) + ": " + hipGetErrorString(e);
    return FLH_ERR_HIP;
}
int num_cus() { return g_cus; }

int launch_zero(void * p, size_t n, hipStream_t s);
int quantize_host(int fmt, const float * src, uint32_t rows, uint32_t cols, uint8_t * dst);

static uint32_t blk_elems(int fmt) {
    switch (fmt) {
        case FLH_FMT_Q8_0: case FLH_FMT_Q5_0: return 32;
        case FLH_FMT_Q4_K: case FLH_FMT_Q6_K: case FLH_FMT_IQ2_XXS: case FLH_FMT_IQ3_XXS: return 256;
        default: return 1;
    }
}
static uint32_t blk_bytes(int fmt) {
    switch (fmt) {
        case FLH_FMT_Q8_0: return 34; case FLH_FMT_Q5_0: return 22; case FLH_FMT_Q4_K: return 144;
        case FLH_FMT_Q6_K: return 210; case FLH_FMT_IQ2_XXS: return 66; case FLH_FMT_IQ3_XXS: return 98;
        default: return 4;
    }
}

static int need_init() {
    if (g_device < 0) return set_error(FLH_ERR_STATE, "flh_init() has not been called");
    return FLH_OK;
}
int need_device() { return need_init(); }

// freeze()-style validation of one dot tile (src/runtime/graph.cpp:84-90)
// Weight address / expert stride alignment: 4 bytes for F32 and Q4_K, 2 for
// the 2-byte aligned block formats (see validate_dot)
static uint64_t w_align_mask(int fmt) { return fmt == FLH_FMT_F32 || fmt == FLH_FMT_Q4_K ? 3 : 1; }

static int validate_dot(int fmt, const void * w, uint64_t w_bytes, uint32_t rows, uint32_t cols,
                        const float * x, float * y, uint32_t nx, const uint32_t * id_slot,
                        uint64_t estride, uint32_t ystride) {
    if (fmt < FLH_FMT_F32 || fmt > FLH_FMT_IQ3_XXS) return set_error(FLH_ERR_ARG, "unknown weight format");
    if (cols % blk_elems(fmt) != 0)
        return set_error(FLH_ERR_ARG, "STREAM_DOT cols not a multiple of the format block size");
    if (w_bytes != (uint64_t)rows * flh_row_bytes(fmt, cols))
        return set_error(FLH_ERR_ARG, "STREAM_DOT w_bytes mismatch");
    if (id_slot && estride == 0) return set_error(FLH_ERR_ARG, "STREAM_DOT_IDX without id slot / stride");
    if (nx > FLH_MAX_DOT_COLS) return set_error(FLH_ERR_ARG, "nx exceeds kMaxDotCols (16)");
    if (rows && (!w || !x || !y)) return set_error(FLH_ERR_ARG, "null weight / activation / output pointer");
    // weights: the 2-byte aligned block formats (Q8_0 34 B, Q5_0 22 B, Q6_K
    // 210 B, IQ) reach any even address (a row tile of a matrix whose rows are
    // 2 mod 4 bytes long); every kernel that needs more alignment declines
    // and the register / fp32 kernels read them through aligned windows
    const uint64_t wal = w_align_mask(fmt);
    if (((uintptr_t)w & wal) || (estride & wal))
        return set_error(FLH_ERR_ARG, "w and the expert stride must be 4-byte aligned (F32, Q4_K) or 2-byte aligned");
    if (((uintptr_t)x & 3) || ((uintptr_t)y & 3)) return set_error(FLH_ERR_ARG, "x and y must be 4-byte aligned");
    // the columns' outputs are computed at once: overlapping ones would race
    // (the reference's CPU loop would accumulate them in turn)
    if (nx > 1 && ystride < rows) return set_error(FLH_ERR_ARG, "multi-column outputs overlap: ystride < rows");
    return FLH_OK;
}

// Several activation columns quantised at once: each column's fp32 values
// and appendices (x_alloc_bytes) must not overlap the next column's.
static int validate_xstride(uint32_t cols, uint32_t nx, uint32_t xstride) {
    if (nx > 1 && (uint64_t)xstride * 4 < x_alloc_bytes(cols))
        return set_error(FLH_ERR_ARG, "act_q8: columns overlap: xstride * 4 < flh_x_alloc_bytes(cols)");
    return FLH_OK;
}

// The launch tuning in force: an immutable Tune published through an atomic
// pointer, so a launch on another thread that runs while flh_init re-reads
// the overrides sees either the old or the new settings, never a mix.  A
// replaced Tune is kept (a few dozen bytes per flh_init call), since a launch
// may still hold a reference to it.
static const Tune g_tune_default{};
static std::atomic<const Tune *> g_tune{&g_tune_default};
const Tune & tune() { return *g_tune.load(std::memory_order_acquire); }

// Development overrides of the launch tuning (see struct Tune).
void load_tune() {
    Tune * tp = new Tune();
    Tune & t = *tp;
    if (const char * e = getenv("FLH_FUSE_MAX_COLS")) t.fuse_max_cols = (uint32_t)strtoul(e, nullptr, 0);
    if (const char * e = getenv("FLH_KS_TUNE")) {
        unsigned a = 0, b = 0, c = 0, d = 0;
        if (sscanf(e, "%u,%u,%u,%u", &a, &b, &c, &d) >= 3) {
            t.ks_wgs_per_cu = a; t.ks_nr = b; t.ks_D = c; t.ks_pro = d;
        }
    }
    if (const char * e = getenv("FLH_KS_W8")) {
        unsigned a = 0, b = 0;
        if (sscanf(e, "%u,%u", &a, &b) == 2) { t.ks_w8_mode = a; t.ks_w8_wgs = b; }
    }
    if (const char * e = getenv("FLH_KQ_TUNE")) {
        unsigned a = 0, b = 0, c = 0;
        if (sscanf(e, "%u,%u,%u", &a, &b, &c) == 3) { t.kq_wgs_per_cu = a; t.kq_nr = b; t.kq_D = c; }
    }
    if (const char * e = getenv("FLH_MFMA_PRO")) t.mf_pro = (uint32_t)atoi(e);
    if (const char * e = getenv("FLH_MFMA_TUNE")) {
        unsigned d = 0, n = 0, k = 0;
        const int got = sscanf(e, "%u,%u,%u", &d, &n, &k);
        if (got >= 2) { t.mf_D = d; t.mf_nrb = n; }
        if (got == 3) t.mf_kh = (int)k;
    }
    if (const char * e = getenv("FLH_MFMA_XC")) t.mf_xc = atoi(e) != 0;
    if (const char * e = getenv("FLH_MFMA_OWN")) t.mf_own = atoi(e) != 0;
    if (const char * e = getenv("FLH_MFMA_MIN_COLS")) t.mf_min_cols = (uint32_t)atoi(e);
    if (const char * e = getenv("FLH_NO_MFMA")) t.no_mfma = atoi(e) != 0;
    if (const char * e = getenv("FLH_NO_Q6MF")) t.no_q6mf = atoi(e) != 0;
    if (const char * e = getenv("FLH_Q6MF_MIN")) {
        unsigned r = 0, c = 0;
        if (sscanf(e, "%u,%u", &r, &c) == 2) { t.q6mf_rows = r; t.q6mf_cols = c; }
    }
    if (const char * e = getenv("FLH_SBL_NX_DEP")) t.sbl_nx_dep = (uint32_t)atoi(e);
    if (const char * e = getenv("FLH_GGUF_THREADS")) t.gguf_threads = (uint32_t)strtoul(e, nullptr, 0);
    if (const char * e = getenv("FLH_SBL")) {
        unsigned on = 1, w = 0, g = 0, m = 0, pre = 0;
        if (sscanf(e, "%u,%u,%u,%u,%u", &on, &w, &g, &m, &pre) >= 1) {
            t.sbl = on; t.sbl_w = w; t.sbl_wpc = g; t.sbl_gmax = m; t.sbl_pre = pre;
        }
    }
    g_tune.store(tp, std::memory_order_release);
}

static int dispatch_dot(int fmt, const DotArgs & a, int fast, uint32_t i8_mask, uint32_t i8k_mask,
                        hipStream_t s) {
    if (!fast) return launch_dot_canonical(fmt, a, s);
    // rows of no columns: every order's dot is +0 (y += 0); the fp32 kernels
    // are the ones planned for it
    if (a.cols == 0) return launch_dot_fast_f32(fmt, a, s);
    if ((fmt == FLH_FMT_Q4_K || fmt == FLH_FMT_Q6_K) && ((i8k_mask >> fmt) & 1u))
        return launch_dot_i8k(fmt, a, s);
    if (fmt != FLH_FMT_F32 && ((i8_mask >> fmt) & 1u)) {
        // 2..8 columns of the 32-weight-block formats: one weight pass on the
        // superblock-per-lane layout where its LDS plan fits
        if (a.nx >= 2 && tune().sbl &&
            (fmt == FLH_FMT_Q8_0 || fmt == FLH_FMT_Q5_0 || fmt == FLH_FMT_IQ2_XXS || fmt == FLH_FMT_IQ3_XXS)) {
            const int rc = launch_dot_sbl_nx(fmt, a, s);
            if (rc != FLH_ERR_UNSUPPORTED) return rc;
        }
        if (fmt == FLH_FMT_Q8_0) {
            const int rc = launch_dot_kstream(fmt, a, s);     // LDS-staged; register kernel otherwise
            return rc != FLH_ERR_UNSUPPORTED ? rc : launch_dot_i8_q8_0(a, s);
        }
        if (fmt == FLH_FMT_Q4_K || fmt == FLH_FMT_Q6_K) return launch_dot_i8_k(fmt, a, s);
        // Q5_0, IQ2_XXS, IQ3_XXS: one column on the LDS-staged kernel where its
        // shape fits, the register kernel otherwise
        if (tune().sbl) {
            const int rc = launch_dot_sbl(fmt, a, false, s);
            if (rc != FLH_ERR_UNSUPPORTED) return rc;
        }
        if (fmt == FLH_FMT_Q5_0) return launch_dot_i8_q5_0(a, s);
        return launch_dot_i8_iq(fmt, a, s);
    }
    return launch_dot_fast_f32(fmt, a, s);
}

// Grouped expert dots of the 32-weight-block formats (Q8_0, Q5_0, IQ2_XXS,
// IQ3_XXS x q8_1): the routed superblock-per-lane launch, one workgroup row
// per (token, slot) pair (the reference runs these per pair too,
// src/model/decoder.cpp:941-996).  Shapes its LDS plan cannot hold (rows of
// more than ~14.5K columns, weights or x not 16-byte aligned) run as the
// reference's own per-pair STREAM_DOT_IDX tiles, the id read on the device,
// on the q8_1 int8 path the routed launch computes (same bits); there the
// ids must be < n_expert, as ROUTER_SEL writes them (the routed launch also
// skips larger ones).
static int launch_moe_b32(int fmt, const MoeArgs & a, hipStream_t s) {
    if (a.rows == 0 || a.ntok == 0 || a.top_k == 0) return FLH_OK;
    if (a.ntok * a.top_k > 256) return set_error(FLH_ERR_UNSUPPORTED, "moe: ntok*top_k > 256");
    const int rc = launch_moe_sbl(fmt, a, s);
    if (rc != FLH_ERR_UNSUPPORTED) return rc;
    for (uint32_t p = 0; p < a.ntok * a.top_k; ++p) {
        const uint32_t xi = a.x_per_slot ? p : p / a.top_k;
        DotArgs d{a.w, a.ids + p, a.estride, a.x + (size_t)xi * a.xstride, a.y + (size_t)p * a.ystride,
                  a.rows, a.cols, 1u, 0u, 0u};
        if (int r = dispatch_dot(fmt, d, 1, 1u << fmt, 0u, s)) return r;
    }
    return FLH_OK;
}

// The decode ops' param blocks are read here, on the host, so they must not
// be plain device memory (reading one would fault the process).  Pointers
// the runtime does not know (ordinary host memory) report an error or
// "unregistered": both are host memory.
static bool host_readable(const void * p) {
    hipPointerAttribute_t at;
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
        (void)hipGetLastError();                                  // not a runtime allocation: host memory
        return true;
    }
    return at.type != hipMemoryTypeDevice && at.type != hipMemoryTypeArray;
}

// freeze()-style validation of a whole task table (nothing is launched on error)
static int validate_table(const flh_task * t, uint32_t n) {
    if (n && !t) return set_error(FLH_ERR_ARG, "null task table");
    for (uint32_t i = 0; i < n; ++i) {
        const flh_task & k = t[i];
        switch (k.kind) {
            case FLH_TASK_STREAM_DOT: case FLH_TASK_STREAM_DOT_IDX: {
                const uint32_t * slot = k.kind == FLH_TASK_STREAM_DOT_IDX ? (const uint32_t *)k.aux : nullptr;
                if (k.kind == FLH_TASK_STREAM_DOT_IDX && (!k.aux || !k.aux2))
                    return set_error(FLH_ERR_ARG, "STREAM_DOT_IDX without id slot / stride");
                if (int rc = validate_dot(k.fmt, k.w, k.w_bytes, k.rows, k.cols, (const float *)k.x,
                                          (float *)k.y, k.nx ? k.nx : 1, slot, k.aux2, k.ystride)) return rc;
                break;
            }
            case FLH_TASK_ACT_Q8:
                if (!k.x || ((uintptr_t)k.x & 15)) return set_error(FLH_ERR_ARG, "ACT_Q8: x must be 16-byte aligned");
                break;
            case FLH_TASK_MERGE: case FLH_TASK_SIGNAL: break;
            case FLH_TASK_ROUTER_SEL: case FLH_TASK_SILU_MUL: case FLH_TASK_WMERGE: case FLH_TASK_RMSNORM:
                if (!k.aux) return set_error(FLH_ERR_ARG, "decode op without aux param block");
                if (!host_readable(k.aux))
                    return set_error(FLH_ERR_ARG, "decode op param block (aux) is in device memory: the host reads "
                                                  "it when the table is issued (use host, pinned or managed memory)");
                break;
            default:
                return set_error(FLH_ERR_UNSUPPORTED, "task kind not supported by the HIP backend");
        }
    }
    return FLH_OK;
}

}  // namespace flh

using namespace flh;

struct flh_arena {
    uint8_t * base;
    size_t cap, used;
};

extern "C" {

const char * flh_last_error(void) { return g_err.c_str(); }

int flh_init(int device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return set_error(FLH_ERR_STATE, "no HIP device visible");
    if (device < 0 || device >= n) return set_error(FLH_ERR_ARG, "device index out of range");
    if (int rc = hip_check(hipSetDevice(device), "hipSetDevice")) return rc;
    hipDeviceProp_t p;
    if (int rc = hip_check(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties")) return rc;
    g_cus = p.multiProcessorCount > 0 ? p.multiProcessorCount : 256;
    g_device = device;
    load_tune();
    return FLH_OK;
}

int flh_device_info(int * num_cus, size_t * hbm_bytes, int * wave_size, char * name, size_t name_len) {
    if (int rc = need_init()) return rc;
    hipDeviceProp_t p;
    if (int rc = hip_check(hipGetDeviceProperties(&p, g_device), "hipGetDeviceProperties")) return rc;
    if (num_cus) *num_cus = p.multiProcessorCount;
    if (hbm_bytes) *hbm_bytes = p.totalGlobalMem;
    if (wave_size) *wave_size = p.warpSize;
    if (name && name_len) {
        strncpy(name, p.gcnArchName, name_len - 1);
        name[name_len - 1] = 0;
    }
    return FLH_OK;
}

int flh_mfma_plan(uint32_t rows, uint32_t cols, uint32_t nx, uint32_t * out) {
    if (int rc = need_init()) return rc;
    if (!out) return set_error(FLH_ERR_ARG, "null plan output");
    return mfma_plan(rows, cols, nx, out);
}

void flh_default_masks(uint32_t * i8_mask, uint32_t * i8k_mask) {
    // kI8MaskCpuDefault / kI8KMaskCpuDefault (src/runtime/kernels.h:920,937)
    if (i8_mask) *i8_mask = (1u << FLH_FMT_Q8_0) | (1u << FLH_FMT_Q5_0) | (1u << FLH_FMT_Q4_K) | (1u << FLH_FMT_Q6_K);
    if (i8k_mask) *i8k_mask = (1u << FLH_FMT_Q4_K) | (1u << FLH_FMT_Q6_K);
}

uint64_t flh_row_bytes(int fmt, uint32_t cols) {
    return (uint64_t)(cols / blk_elems(fmt)) * blk_bytes(fmt);
}
size_t flh_x_alloc_bytes(uint32_t cols) { return flh::x_alloc_bytes(cols); }

// ---------------------------------------------------------------- memory --
int flh_arena_create(size_t bytes, flh_arena ** out) {
    if (int rc = need_init()) return rc;
    if (!out) return set_error(FLH_ERR_ARG, "null out");
    void * p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 256) != hipSuccess)
        return set_error(FLH_ERR_NOMEM, "arena hipMalloc failed");
    *out = new flh_arena{(uint8_t *)p, bytes, 0};
    return FLH_OK;
}
int flh_arena_alloc(flh_arena * a, size_t bytes, size_t align, void ** out) {
    if (!a || !out) return set_error(FLH_ERR_ARG, "null arena / out");
    if (align < 16) align = 16;
    if (align & (align - 1)) return set_error(FLH_ERR_ARG, "alignment must be a power of two");
    // aligned as an address (the base is only as aligned as hipMalloc makes it)
    const uintptr_t base = (uintptr_t)a->base, at = base + a->used;
    if (at > UINTPTR_MAX - (align - 1)) return set_error(FLH_ERR_NOMEM, "arena exhausted");
    const size_t off = (size_t)(((at + align - 1) & ~(uintptr_t)(align - 1)) - base);
    if (off > a->cap || bytes > a->cap - off) return set_error(FLH_ERR_NOMEM, "arena exhausted");
    a->used = off + bytes;
    *out = a->base + off;
    return FLH_OK;
}
size_t flh_arena_used(const flh_arena * a) { return a ? a->used : 0; }
int flh_arena_destroy(flh_arena * a) {
    if (!a) return FLH_OK;
    const int rc = hip_check(hipFree(a->base), "arena hipFree");
    delete a;
    return rc;
}
int flh_malloc(size_t bytes, void ** out) {
    if (int rc = need_init()) return rc;
    if (!out) return set_error(FLH_ERR_ARG, "null out");
    if (hipMalloc(out, bytes ? bytes : 256) != hipSuccess) return set_error(FLH_ERR_NOMEM, "hipMalloc failed");
    return FLH_OK;
}
int flh_host_alloc(size_t bytes, void ** out) {
    if (int rc = need_init()) return rc;
    if (!out) return set_error(FLH_ERR_ARG, "null out");
    if (hipHostMalloc(out, bytes ? bytes : 256, hipHostMallocDefault) != hipSuccess)
        return set_error(FLH_ERR_NOMEM, "hipHostMalloc failed");
    return FLH_OK;
}
int flh_host_free(void * p) { return p ? hip_check(hipHostFree(p), "hipHostFree") : FLH_OK; }
int flh_free(void * p) { return p ? hip_check(hipFree(p), "hipFree") : FLH_OK; }
int flh_upload(void * dst, const void * src, size_t n, void * stream) {
    if (int rc = hip_check(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, (hipStream_t)stream), "upload")) return rc;
    return hip_check(hipStreamSynchronize((hipStream_t)stream), "upload sync");
}
int flh_download(void * dst, const void * src, size_t n, void * stream) {
    if (int rc = hip_check(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, (hipStream_t)stream), "download")) return rc;
    return hip_check(hipStreamSynchronize((hipStream_t)stream), "download sync");
}
int flh_copy(void * dst, const void * src, size_t n, void * stream) {
    return hip_check(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, (hipStream_t)stream), "copy");
}
int flh_zero(void * dst, size_t n, void * stream) { return launch_zero(dst, n, (hipStream_t)stream); }

// --------------------------------------------------------------- streams --
int flh_stream_create(void ** out) {
    if (int rc = need_init()) return rc;
    if (!out) return set_error(FLH_ERR_ARG, "null out");
    hipStream_t s;
    if (int rc = hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate")) return rc;
    *out = (void *)s;
    return FLH_OK;
}
int flh_stream_sync(void * s) { return hip_check(hipStreamSynchronize((hipStream_t)s), "hipStreamSynchronize"); }
int flh_stream_destroy(void * s) { return s ? hip_check(hipStreamDestroy((hipStream_t)s), "hipStreamDestroy") : FLH_OK; }
int flh_event_create(void ** out) {
    if (!out) return set_error(FLH_ERR_ARG, "null out");
    hipEvent_t e;
    if (int rc = hip_check(hipEventCreate(&e), "hipEventCreate")) return rc;
    *out = (void *)e;
    return FLH_OK;
}
int flh_event_record(void * e, void * s) { return hip_check(hipEventRecord((hipEvent_t)e, (hipStream_t)s), "hipEventRecord"); }
int flh_event_elapsed_ms(void * a, void * b, float * ms) {
    if (!ms) return set_error(FLH_ERR_ARG, "null ms");
    if (int rc = hip_check(hipEventSynchronize((hipEvent_t)b), "hipEventSynchronize")) return rc;
    return hip_check(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b), "hipEventElapsedTime");
}
int flh_event_destroy(void * e) { return e ? hip_check(hipEventDestroy((hipEvent_t)e), "hipEventDestroy") : FLH_OK; }

// ---------------------------------------------------------------- graphs --
int flh_graph_capture_begin(void * stream) {
    if (int rc = need_init()) return rc;
    return hip_check(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal),
                     "hipStreamBeginCapture");
}
int flh_graph_capture_end(void * stream, void ** graph_exec) {
    hipGraph_t g = nullptr;
    // (with a null graph_exec the capture still ends, so the stream is usable)
    if (int rc = hip_check(hipStreamEndCapture((hipStream_t)stream, &g), "hipStreamEndCapture")) return rc;
    hipGraphExec_t ge = nullptr;
    if (!graph_exec) {
        (void)hipGraphDestroy(g);
        return set_error(FLH_ERR_ARG, "null graph_exec");
    }
    const int rc = hip_check(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    if (rc) return rc;
    *graph_exec = (void *)ge;
    return FLH_OK;
}
int flh_graph_launch(void * ge, void * stream) {
    return hip_check(hipGraphLaunch((hipGraphExec_t)ge, (hipStream_t)stream), "hipGraphLaunch");
}
int flh_graph_destroy(void * ge) {
    return ge ? hip_check(hipGraphExecDestroy((hipGraphExec_t)ge), "hipGraphExecDestroy") : FLH_OK;
}

// ------------------------------------------------------------------- ops --
int flh_act_q8(float * x, void * y_q81, uint32_t cols, uint32_t nx, uint32_t xstride, void * stream) {
    if (int rc = need_init()) return rc;
    if (nx == 0) nx = 1;
    if (!x || ((uintptr_t)x & 15) || (nx > 1 && (xstride & 3)))
        return set_error(FLH_ERR_ARG, "act_q8: x must be non-null and 16-byte aligned, xstride a multiple of 4");
    if (y_q81 && ((uintptr_t)y_q81 & 3)) return set_error(FLH_ERR_ARG, "act_q8: y must be 4-byte aligned");
    if (int rc = validate_xstride(cols, nx, xstride)) return rc;
    return launch_act_q8(x, y_q81, cols, nx, xstride, (hipStream_t)stream);
}

int flh_stream_dot(int fmt, const void * w, uint64_t w_bytes, uint32_t rows, uint32_t cols,
                   const float * x, float * y, uint32_t nx, uint32_t xstride, uint32_t ystride,
                   const uint32_t * id_slot, uint64_t estride, int fast, uint32_t i8_mask,
                   uint32_t i8k_mask, void * stream) {
    if (nx == 0) nx = 1;
    if (int rc = validate_dot(fmt, w, w_bytes, rows, cols, x, y, nx, id_slot, estride, ystride)) return rc;
    if (int rc = need_init()) return rc;
    DotArgs a{(const uint8_t *)w, id_slot, estride, x, y, rows, cols, nx, xstride, ystride};
    return dispatch_dot(fmt, a, fast, i8_mask, i8k_mask, (hipStream_t)stream);
}

int flh_act_q8_stream_dot(int fmt, const void * w, uint64_t w_bytes, uint32_t rows, uint32_t cols,
                          float * x, float * y, uint32_t nx, uint32_t xstride, uint32_t ystride,
                          const uint32_t * id_slot, uint64_t estride, int fast, uint32_t i8_mask,
                          uint32_t i8k_mask, void * stream) {
    if (nx == 0) nx = 1;
    if (int rc = validate_dot(fmt, w, w_bytes, rows, cols, x, y, nx, id_slot, estride, ystride)) return rc;
    if (((uintptr_t)x & 15) || (nx > 1 && (xstride & 3)))
        return set_error(FLH_ERR_ARG, "act_q8: x must be 16-byte aligned, xstride a multiple of 4");
    if (int rc = validate_xstride(cols, nx, xstride)) return rc;
    if (int rc = need_init()) return rc;
    hipStream_t s = (hipStream_t)stream;
    DotArgs a{(const uint8_t *)w, id_slot, estride, x, y, rows, cols, nx, xstride, ystride};
    // Fused when every workgroup re-reading the fp32 column is cheaper than a
    // separate ACT_Q8 launch.
    if (fast && cols > 0 && cols <= tune().fuse_max_cols && (fmt == FLH_FMT_Q4_K || fmt == FLH_FMT_Q6_K) && ((i8k_mask >> fmt) & 1u)) {
        const int rc = launch_act_dot_kstream(fmt, a, s);
        if (rc != FLH_ERR_UNSUPPORTED) return rc;
    }
    if (int rc = launch_act_q8(x, nullptr, cols, nx, xstride, s)) return rc;
    return dispatch_dot(fmt, a, fast, i8_mask, i8k_mask, s);
}

// RMSNORM -> ACT_Q8 -> one-column dot in one launch where the superblock-per-
// lane kernel takes it (Q4_K on the int8 path), else the two calls.
static int rmsnorm_dot(int fmt, const DotArgs & a, const NormArgs & nm, int fast, uint32_t i8_mask,
                       uint32_t i8k_mask, hipStream_t s) {
    const float * xb = nm.x, * xe = nm.x + a.cols;
    const float * yb = a.x, * ye = (const float *)((const uint8_t *)a.x + x_alloc_bytes(a.cols));
    const bool overlap = xb < ye && yb < xe;
    if (fast && !overlap && fmt == FLH_FMT_Q4_K && ((i8k_mask >> fmt) & 1u) && a.cols > 0 && a.cols <= 8192) {
        // the kernel the plain fused ACT_Q8 dot takes at this size (above 2^18
        // superblocks the four-lanes one)
        int rc = FLH_ERR_UNSUPPORTED;
        if ((uint64_t)a.rows * (a.cols >> 8) > (1u << 18) || !tune().sbl) rc = launch_norm_dot_kstream(a, nm, s);
        if (rc == FLH_ERR_UNSUPPORTED && tune().sbl) rc = launch_dot_sbl(fmt, a, true, s, &nm);
        if (rc != FLH_ERR_UNSUPPORTED) return rc;
    }
    if (int rc = launch_rmsnorm_act_q8(nm.x, nm.wn, (float *)a.x, a.cols, nm.eps, true, s)) return rc;
    return dispatch_dot(fmt, a, fast, i8_mask, i8k_mask, s);
}

int flh_rmsnorm_stream_dot(int fmt, const void * w, uint64_t w_bytes, uint32_t rows, uint32_t cols, const float * x,
                           const float * wnorm, float eps, float * xn, float * y, int fast, uint32_t i8_mask,
                           uint32_t i8k_mask, void * stream) {
    if (int rc = validate_dot(fmt, w, w_bytes, rows, cols, xn, y, 1, nullptr, 0, 0)) return rc;
    if (!x || !wnorm || ((uintptr_t)x & 15) || ((uintptr_t)wnorm & 15) || ((uintptr_t)xn & 15))
        return set_error(FLH_ERR_ARG, "rmsnorm dot: x, wnorm, xn non-null and 16-byte aligned");
    if (cols % 256) return set_error(FLH_ERR_ARG, "rmsnorm dot: cols must be a multiple of 256 (the q8_K appendix)");
    if (int rc = need_init()) return rc;
    const float * xe = x + cols;
    const float * ye = (const float *)((const uint8_t *)xn + x_alloc_bytes(cols));
    if (x < ye && xn < xe) return set_error(FLH_ERR_ARG, "rmsnorm dot: xn overlaps x");
    DotArgs a{(const uint8_t *)w, nullptr, 0, xn, y, rows, cols, 1u, 0, 0};
    return rmsnorm_dot(fmt, a, NormArgs{x, wnorm, eps}, fast, i8_mask, i8k_mask, (hipStream_t)stream);
}

int flh_dequant(int fmt, const void * w, uint32_t rows, uint32_t cols, float * out, void * stream) {
    if (int rc = need_init()) return rc;
    if (cols % blk_elems(fmt)) return set_error(FLH_ERR_ARG, "dequant: cols not a multiple of the block size");
    return launch_dequant(fmt, (const uint8_t *)w, rows, cols, out, (hipStream_t)stream);
}

int flh_exec_tasks(const flh_task * t, uint32_t n, int fast, uint32_t i8_mask, uint32_t i8k_mask,
                   void * stream) {
    if (int rc = validate_table(t, n)) return rc;
    if (int rc = need_init()) return rc;
    hipStream_t s = (hipStream_t)stream;
    for (uint32_t i = 0; i < n; ++i) {
        const flh_task & k = t[i];
        int rc = FLH_OK;
        switch (k.kind) {
            case FLH_TASK_STREAM_DOT: case FLH_TASK_STREAM_DOT_IDX: {
                const bool idx = k.kind == FLH_TASK_STREAM_DOT_IDX;
                DotArgs a{(const uint8_t *)k.w, idx ? (const uint32_t *)k.aux : nullptr, idx ? k.aux2 : 0,
                          (const float *)k.x, (float *)k.y, k.rows, k.cols, k.nx ? k.nx : 1u,
                          k.xstride, k.ystride};
                // fuse following row tiles of the same matrix into this launch
                while (i + 1 < n) {
                    const flh_task & q = t[i + 1];
                    if (q.kind != k.kind || q.fmt != k.fmt || q.cols != k.cols || q.x != k.x ||
                        (q.nx ? q.nx : 1u) != a.nx || q.xstride != k.xstride || q.ystride != k.ystride ||
                        q.aux != k.aux || q.aux2 != k.aux2 ||
                        (const uint8_t *)q.w != a.w + (uint64_t)a.rows * flh_row_bytes(k.fmt, k.cols) ||
                        (float *)q.y != a.y + a.rows || (a.nx > 1 && a.rows + q.rows > k.ystride))
                        break;
                    a.rows += q.rows;
                    ++i;
                }
                rc = dispatch_dot(k.fmt, a, fast, i8_mask, i8k_mask, s);
                break;
            }
            case FLH_TASK_ACT_Q8: {
                // ACT_Q8 whose next task is a single-column q8_K dot of the
                // same activation: one fused launch (same appendix bytes,
                // same outputs).
                const flh_task * q = i + 1 < n ? &t[i + 1] : nullptr;
                const bool canon_y = (const uint8_t *)k.y == (const uint8_t *)k.x + xq_off(k.cols);
                if (q && canon_y && fast && k.cols <= tune().fuse_max_cols && q->kind == FLH_TASK_STREAM_DOT && q->x == k.x &&
                    q->cols == k.cols && (q->nx ? q->nx : 1u) == 1 &&
                    (q->fmt == FLH_FMT_Q4_K || q->fmt == FLH_FMT_Q6_K) && ((i8k_mask >> q->fmt) & 1u)) {
                    DotArgs a{(const uint8_t *)q->w, nullptr, 0, (const float *)q->x, (float *)q->y,
                              q->rows, q->cols, 1u, q->xstride, q->ystride};
                    rc = launch_act_dot_kstream(q->fmt, a, s);
                    if (rc != FLH_ERR_UNSUPPORTED) {
                        ++i;
                        break;
                    }
                }
                rc = launch_act_q8((float *)k.x, k.y, k.cols, 1, 0, s);
                break;
            }
            case FLH_TASK_MERGE:
                rc = launch_merge((const float *)k.x, (float *)k.y, k.rows, k.cols, s);
                break;
            case FLH_TASK_SIGNAL: break;
            case FLH_TASK_RMSNORM: {
                const flh_rmsnorm_p & p = *(const flh_rmsnorm_p *)k.aux;
                // RMSNORM followed by the ACT_Q8 of its output (the decoder's
                // norm -> quant chain): one launch
                const flh_task * q = i + 1 < n ? &t[i + 1] : nullptr;
                const bool fuse = q && q->kind == FLH_TASK_ACT_Q8 && q->x == (const void *)p.y && q->cols == p.n &&
                                  (const uint8_t *)q->y == (const uint8_t *)p.y + xq_off(p.n) &&
                                  !((uintptr_t)p.y & 15);
                // ... and a single-column dot of that activation: one launch
                const flh_task * d = fuse && i + 2 < n ? &t[i + 2] : nullptr;
                if (d && d->kind == FLH_TASK_STREAM_DOT && d->x == (const void *)p.y && d->cols == p.n &&
                    (d->nx ? d->nx : 1u) == 1 && p.n % 256 == 0 && !((uintptr_t)p.x & 15) &&
                    !((uintptr_t)p.wnorm & 15)) {
                    DotArgs a{(const uint8_t *)d->w, nullptr, 0, (const float *)d->x, (float *)d->y, d->rows, d->cols,
                              1u, d->xstride, d->ystride};
                    rc = rmsnorm_dot(d->fmt, a, NormArgs{p.x, p.wnorm, p.eps}, fast, i8_mask, i8k_mask, s);
                    i += 2;
                    break;
                }
                rc = launch_rmsnorm_act_q8(p.x, p.wnorm, p.y, p.n, p.eps, fuse, s);
                if (fuse) ++i;
                break;
            }
            case FLH_TASK_ROUTER_SEL: {
                const flh_router_p & p = *(const flh_router_p *)k.aux;
                rc = launch_router_sel(p.logits, 1, p.n_expert, p.top_k, p.norm, p.scale, p.ids, p.gates, s);
                break;
            }
            case FLH_TASK_SILU_MUL: {
                const flh_silu_mul_p & p = *(const flh_silu_mul_p *)k.aux;
                // SILU_MUL followed by the ACT_Q8 of its output (the
                // decoder's down-projection input): one fused launch
                const flh_task * q = i + 1 < n ? &t[i + 1] : nullptr;
                if (q && q->kind == FLH_TASK_ACT_Q8 && q->x == (void *)p.h && q->cols == p.n &&
                    (const uint8_t *)q->y == (const uint8_t *)p.h + xq_off(p.n) && !((uintptr_t)p.h & 15)) {
                    rc = launch_silu_act_q8(p.gate, p.up, p.h, p.n, 1, 0, 0, s);
                    ++i;
                    break;
                }
                rc = launch_silu_mul(p.gate, p.up, p.h, p.n, 1, 0, 0, s);
                break;
            }
            case FLH_TASK_WMERGE: {
                const flh_wmerge_p & p = *(const flh_wmerge_p *)k.aux;
                rc = launch_wmerge(p.parts, p.gates, p.add1, p.add2, p.y, p.scale, p.n_parts, p.n,
                                   p.n_full, 1, 0, 0, s);
                break;
            }
        }
        if (rc) return rc;
    }
    return FLH_OK;
}

// ------------------------------------------------------------------- MoE --
int flh_moe_dot(int fmt, const void * w, uint64_t estride, uint32_t rows, uint32_t cols,
                const uint32_t * ids, uint32_t ntok, uint32_t top_k, uint32_t n_expert,
                const float * x, uint32_t xstride, uint32_t x_per_slot, float * y, uint32_t ystride,
                void * stream) {
    if (int rc = need_init()) return rc;
    if (fmt < FLH_FMT_Q8_0 || fmt > FLH_FMT_IQ3_XXS)
        return set_error(FLH_ERR_UNSUPPORTED, "moe_dot: quantized weight formats only");
    if (cols % 256 || cols == 0) return set_error(FLH_ERR_ARG, "moe_dot: cols not a positive multiple of 256");
    if (!w || !ids || !x || !y || n_expert == 0) return set_error(FLH_ERR_ARG, "moe_dot: null argument");
    if (estride < (uint64_t)rows * flh_row_bytes(fmt, cols) || (estride & w_align_mask(fmt)) ||
        ((uintptr_t)w & w_align_mask(fmt)))
        return set_error(FLH_ERR_ARG, "moe_dot: expert stride smaller than one expert or misaligned");
    MoeArgs a{(const uint8_t *)w, estride, ids, x, y, rows, cols, ntok, top_k, n_expert, xstride, ystride,
              x_per_slot};
    if (fmt == FLH_FMT_Q4_K || fmt == FLH_FMT_Q6_K) return launch_moe_i8k(fmt, a, (hipStream_t)stream);
    return launch_moe_b32(fmt, a, (hipStream_t)stream);
}

int flh_router_moe_dot(int fmt, const void * w, uint64_t estride, uint32_t rows, uint32_t cols,
                       const float * logits, uint32_t ntok, uint32_t n_expert, uint32_t top_k, uint32_t norm,
                       float scale, uint32_t * ids, float * gates, const float * x, uint32_t xstride,
                       uint32_t x_per_slot, float * y, uint32_t ystride, void * stream) {
    if (int rc = need_init()) return rc;
    if (fmt < FLH_FMT_Q8_0 || fmt > FLH_FMT_IQ3_XXS)
        return set_error(FLH_ERR_UNSUPPORTED, "router_moe_dot: quantized weight formats only");
    const bool kf = fmt == FLH_FMT_Q4_K || fmt == FLH_FMT_Q6_K;
    if (cols % 256 || cols == 0) return set_error(FLH_ERR_ARG, "router_moe_dot: cols not a positive multiple of 256");
    if (!w || !logits || !ids || !gates || !x || !y || n_expert == 0 || top_k == 0 || top_k > n_expert)
        return set_error(FLH_ERR_ARG, "router_moe_dot: null argument or top_k outside 1..n_expert");
    if (estride < (uint64_t)rows * flh_row_bytes(fmt, cols) || (estride & w_align_mask(fmt)) ||
        ((uintptr_t)w & w_align_mask(fmt)))
        return set_error(FLH_ERR_ARG, "router_moe_dot: expert stride smaller than one expert or misaligned");
    if (ntok == 0) return FLH_OK;
    hipStream_t s = (hipStream_t)stream;
    MoeArgs a{(const uint8_t *)w, estride, ids, x, y, rows, cols, ntok, top_k, n_expert, xstride, ystride,
              x_per_slot};
    // routing inside the grouped kernels (one launch) where they take it
    if (n_expert <= 64 && top_k <= 8 && ntok * top_k <= 256) {
        MoeArgs f = a;
        f.rt_logits = logits;
        f.rt_norm = norm;
        f.rt_scale = scale;
        f.rt_gates = gates;
        int rc = FLH_ERR_UNSUPPORTED;
        if ((ntok == 1 || !kf) && tune().sbl) rc = launch_moe_sbl(fmt, f, s);
        if (rc == FLH_ERR_UNSUPPORTED && kf) rc = launch_moe_mfma(fmt, f, s);
        if (rc == FLH_ERR_UNSUPPORTED && kf) rc = launch_moe_kstream(fmt, f, s);
        if (rc != FLH_ERR_UNSUPPORTED) return rc;
    }
    if (int rc = launch_router_sel(logits, ntok, n_expert, top_k, norm, scale, ids, gates, s)) return rc;
    return kf ? launch_moe_i8k(fmt, a, s) : launch_moe_b32(fmt, a, s);
}

int flh_router_sel(const float * logits, uint32_t ntok, uint32_t n_expert, uint32_t top_k, uint32_t norm,
                   float scale, uint32_t * ids, float * gates, void * stream) {
    if (int rc = need_init()) return rc;
    return launch_router_sel(logits, ntok, n_expert, top_k, norm, scale, ids, gates, (hipStream_t)stream);
}
int flh_silu_mul(const float * gate, const float * up, float * h, uint32_t n, uint32_t ncol,
                 uint32_t gstride, uint32_t hstride, void * stream) {
    if (int rc = need_init()) return rc;
    return launch_silu_mul(gate, up, h, n, ncol, gstride, hstride, (hipStream_t)stream);
}
int flh_rmsnorm_act_q8(const float * x, const float * wnorm, float * y, uint32_t n, float eps, int write_app,
                       void * stream) {
    if (int rc = need_init()) return rc;
    if (!x || !wnorm || !y || ((uintptr_t)x & 3) || ((uintptr_t)wnorm & 3) || ((uintptr_t)y & (write_app ? 15 : 3)))
        return set_error(FLH_ERR_ARG, "rmsnorm: x, wnorm, y non-null and aligned (y 16 bytes with ACT_Q8)");
    return launch_rmsnorm_act_q8(x, wnorm, y, n, eps, write_app != 0, (hipStream_t)stream);
}

int flh_silu_mul_act_q8(const float * gate, const float * up, float * h, uint32_t n, uint32_t ncol,
                        uint32_t gstride, uint32_t hstride, void * stream) {
    if (int rc = need_init()) return rc;
    if (!gate || !up || !h || ((uintptr_t)h & 15) || (ncol > 1 && (hstride & 3)))
        return set_error(FLH_ERR_ARG, "silu_mul_act_q8: h must be 16-byte aligned, hstride a multiple of 4");
    return launch_silu_act_q8(gate, up, h, n, ncol, gstride, hstride, (hipStream_t)stream);
}
int flh_wmerge(const float * parts, const float * gates, const float * add1, const float * add2, float * y,
               float scale, uint32_t n_parts, uint32_t n, uint32_t n_full, uint32_t ncol, uint32_t pstride,
               uint32_t ystride, void * stream) {
    if (int rc = need_init()) return rc;
    return launch_wmerge(parts, gates, add1, add2, y, scale, n_parts, n, n_full, ncol, pstride, ystride,
                         (hipStream_t)stream);
}

// ------------------------------------------------------- synthetic inputs --
int flh_fill_normal(float * dst, size_t n, uint64_t seed, float mean, float stddev, float outlier_frac,
                    float outlier_scale, void * stream) {
    if (int rc = need_init()) return rc;
    return launch_fill_normal(dst, n, seed, mean, stddev, outlier_frac, outlier_scale, (hipStream_t)stream);
}
int flh_quantize(int fmt, const float * src, uint32_t rows, uint32_t cols, void * dst, void * stream) {
    if (int rc = need_init()) return rc;
    return launch_quantize_weights(fmt, src, rows, cols, (uint8_t *)dst, (hipStream_t)stream);
}
int flh_quantize_host(int fmt, const float * src, uint32_t rows, uint32_t cols, void * dst) {
    return quantize_host(fmt, src, rows, cols, (uint8_t *)dst);
}

}  // extern "C"
