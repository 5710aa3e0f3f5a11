/*
 * fastllm_hip.h -- C-ABI of the MI355X (gfx950) quantized-matvec backend.
 *
 * Drop-in for the reference runtime's CUDA execution path of the quantized
 * decode hot path (qdox-labs/fast-llm): the ACT_Q8 / STREAM_DOT /
 * STREAM_DOT_IDX task kinds and the GGUF Q8_0 / Q4_K / Q6_K row-dots behind
 * them.  Plain C types only: device pointers are void* / float*, streams and
 * events are opaque void* (hipStream_t / hipEvent_t), sizes are integers.
 *
 * Every entry point returns FLH_OK (0) or a negative FLH_ERR_* code and
 * records a message readable with flh_last_error() (per calling thread).
 * The reference aborts on every error (src/runtime/gpu_exec.cu:15-17,
 * src/runtime/graph.cpp:100-103); a host wrapper that wants that behaviour
 * aborts on a non-zero return.
 *
 * Numerics contract: with fast=1 and the reference default masks, every
 * STREAM_DOT output is BITWISE equal to the reference CPU int8 path
 * (src/runtime/kernels.h:1002-1258 on x86: fl_dot_i8_q8_0, fl_dot_i8k_q4_K,
 * fl_dot_i8k_q6_K), ACT_Q8 bytes equal fl_exec_act_q8, and flh_dequant
 * equals dequant_chunk (src/runtime/kernels.h:162-242).
 */
#ifndef FASTLLM_HIP_H
#define FASTLLM_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- codes -- */
enum {
    FLH_OK = 0,
    FLH_ERR_ARG = -1,          /* invalid argument (freeze()-style validation) */
    FLH_ERR_HIP = -2,          /* HIP runtime error */
    FLH_ERR_UNSUPPORTED = -3,  /* task kind / format / shape not implemented */
    FLH_ERR_NOMEM = -4,        /* arena exhausted or hipMalloc failed */
    FLH_ERR_STATE = -5,        /* flh_init not called / no device */
    FLH_ERR_IO = -6,           /* file missing or unreadable (GGUF) */
    FLH_ERR_FORMAT = -7        /* malformed GGUF file */
};

/* TaskKind values (include/fastllm/fastllm.h:19-45), stable. */
enum {
    FLH_TASK_STREAM_DOT = 0, FLH_TASK_MERGE = 1, FLH_TASK_SIGNAL = 2,
    FLH_TASK_ACT_Q8 = 3, FLH_TASK_STREAM_DOT_IDX = 4, FLH_TASK_RMSNORM = 5,
    FLH_TASK_ADD2 = 6, FLH_TASK_ROPE_DS2 = 7, FLH_TASK_KV_APPEND = 8,
    FLH_TASK_ATTN_HEAD = 9, FLH_TASK_ROUTER_SEL = 10, FLH_TASK_SILU_MUL = 11,
    FLH_TASK_WMERGE = 12
};

/* Fmt values (include/fastllm/fastllm.h:56-57), stable. */
enum {
    FLH_FMT_F32 = 0, FLH_FMT_Q8_0 = 1, FLH_FMT_Q5_0 = 2, FLH_FMT_Q4_K = 3,
    FLH_FMT_Q6_K = 4, FLH_FMT_IQ2_XXS = 5, FLH_FMT_IQ3_XXS = 6
};

/* Max activation columns per multi-column tile (fastllm.h:61 kMaxDotCols). */
#define FLH_MAX_DOT_COLS 16u

/*
 * Task record, byte-for-byte the layout of fastllm::Task
 * (include/fastllm/fastllm.h:65-97; enum class members are uint8_t), so a
 * frozen graph's task table can be passed as-is.  Pointers w / x / y / aux
 * are DEVICE pointers here (the reference uses unified memory), except that
 * for ROUTER_SEL / SILU_MUL / WMERGE aux points to a HOST-readable param
 * block (flh_router_p etc.) whose own pointers are device pointers.
 */
typedef struct __attribute__((aligned(128))) flh_task {
    uint32_t id;
    uint8_t kind;              /* FLH_TASK_* */
    uint8_t affinity;
    uint8_t fmt;               /* FLH_FMT_* */
    uint16_t n_consumers;
    uint32_t consumers[6];
    const void * w;
    uint64_t w_bytes;
    const void * x;
    void * y;
    uint32_t rows, cols;
    int32_t dep_init;
    int32_t dep_count;
    uint32_t epoch;
    uint64_t handoff_ts;
    const void * aux;          /* STREAM_DOT_IDX: device u32 expert-id slot */
    uint64_t aux2;             /* STREAM_DOT_IDX: expert stride in bytes */
    uint32_t nx, xstride, ystride;
} flh_task;

/* Decode-op param blocks, layouts of RmsNormP / RouterP / SiluMulP / WmergeP
 * (src/runtime/decode_params.h:23-29, 68-97). */
typedef struct flh_rmsnorm_p {
    const float * wnorm; const float * x; float * y; float eps; uint32_t n;
} flh_rmsnorm_p;
typedef struct flh_router_p {
    const float * logits; uint32_t * ids; float * gates;
    uint32_t n_expert, top_k, norm; float scale;
} flh_router_p;
typedef struct flh_silu_mul_p {
    const float * gate; const float * up; float * h; uint32_t n;
} flh_silu_mul_p;
typedef struct flh_wmerge_p {
    const float * parts; const float * gates; const float * add1;
    const float * add2; float * y; float scale; uint32_t n_parts, n, n_full;
} flh_wmerge_p;

/* ------------------------------------------------------------- runtime -- */
/* Last error message of the calling thread ("" if none). */
const char * flh_last_error(void);

/* Select and initialise a device; must precede every call below that touches
 * the GPU.  Replaces the device setup inside gpu_start()
 * (src/runtime/gpu_exec.cu:457-496; prototype runtime_internal.h:292).
 * Each call also (re-)reads the launch-tuning overrides FLH_* from the
 * environment (development sweeps; the defaults are the measured best); no
 * launch reads the environment itself. */
int flh_init(int device);

/* Device facts: compute units, HBM bytes, wave size, name. */
int flh_device_info(int * num_cus, size_t * hbm_bytes, int * wave_size,
                    char * name, size_t name_len);

/* Launch plan of the multi-column matrix-core dot for a Q4_K matrix of
 * rows x cols with nx activation columns on this device: out[0] = K halves,
 * out[1] = activations carried in the chunk DMA, out[2] = rows per batch,
 * out[3] = ring depth.  FLH_ERR_UNSUPPORTED if that kernel does not take the
 * shape.  No counterpart in the reference (whose multi-column kernel has one
 * plan): a query for tests and tuning, launches nothing. */
int flh_mfma_plan(uint32_t rows, uint32_t cols, uint32_t nx, uint32_t * out);

/* Reference default dispatch masks for the CPU int8 path this backend
 * matches (src/runtime/kernels.h:920,937). */
void flh_default_masks(uint32_t * i8_mask, uint32_t * i8k_mask);

/* Row bytes of a weight row and the activation buffer size with both q8
 * appendices (src/runtime/quants.h:97-99, 326-330). */
uint64_t flh_row_bytes(int fmt, uint32_t cols);
size_t flh_x_alloc_bytes(uint32_t cols);

/* ------------------------------------------------------------- memory -- */
/* Device bump arena over one hipMalloc: replaces Arena::create's
 * cudaMallocManaged arena (src/runtime/arena.cpp:54-74).  Allocations are
 * never freed individually; destroy releases everything. */
typedef struct flh_arena flh_arena;
int flh_arena_create(size_t bytes, flh_arena ** out);
int flh_arena_alloc(flh_arena * a, size_t bytes, size_t align, void ** out);
size_t flh_arena_used(const flh_arena * a);
int flh_arena_destroy(flh_arena * a);

/* Plain device buffers (outside any arena). */
int flh_malloc(size_t bytes, void ** out);
int flh_free(void * p);
/* Pinned host memory (hipHostMalloc): host-readable and device-visible; the
 * place for the decode-op param blocks a task table points to (see
 * flh_exec_tasks).  No counterpart in the reference, whose managed arena
 * is host-readable as it is (src/runtime/arena.cpp:54-63). */
int flh_host_alloc(size_t bytes, void ** out);
int flh_host_free(void * p);
int flh_upload(void * dst_dev, const void * src_host, size_t n, void * stream);
int flh_download(void * dst_host, const void * src_dev, size_t n, void * stream);
/* device-to-device copy of n bytes on a stream (asynchronous) */
int flh_copy(void * dst_dev, const void * src_dev, size_t n, void * stream);
/* zero n bytes with a fill kernel (safe inside HIP graph capture) */
int flh_zero(void * dst_dev, size_t n, void * stream);

/* ------------------------------------------------------------ streams -- */
/* Replaces gpu_make_stream / gpu_stop_sync (src/runtime/gpu_exec.cu:387,498).
 * Streams are created at default priority. */
int flh_stream_create(void ** out);
int flh_stream_sync(void * stream);
int flh_stream_destroy(void * stream);
int flh_event_create(void ** out);
int flh_event_record(void * event, void * stream);
int flh_event_elapsed_ms(void * start, void * stop, float * ms);
int flh_event_destroy(void * event);

/* HIP graph capture of work issued on one stream (replaces the reference's
 * persistent-kernel launch amortisation, src/runtime/gpu_exec.cu:156-344,
 * for a frozen graph: capture once, replay per token).  Every kernel of
 * this library is capture-safe (no hipMemsetAsync, no host syncs). */
int flh_graph_capture_begin(void * stream);
int flh_graph_capture_end(void * stream, void ** graph_exec);
int flh_graph_launch(void * graph_exec, void * stream);
int flh_graph_destroy(void * graph_exec);

/* ---------------------------------------------------------------- ops -- */
/* ACT_Q8 (TaskKind 3; fl_exec_act_q8, src/runtime/quants.h:404-416; GPU
 * gact_q8, src/runtime/kernels_gpu.h:881-891): for each of nx columns
 * x_p = x + p*xstride (16-B aligned, fl_x_alloc_bytes(cols) bytes each),
 * write the q8_1 appendix at y_q81 + p*xstride floats (NULL = the canonical
 * fl_xq_of(x_p, cols)) and the q8_K appendix at fl_xqk_of(x_p, cols).
 * nx > 1: columns are quantised at once, so xstride * 4 >= fl_x_alloc_bytes
 * (cols) (FLH_ERR_ARG otherwise). */
int flh_act_q8(float * x, void * y_q81, uint32_t cols, uint32_t nx,
               uint32_t xstride, void * stream);

/* STREAM_DOT / STREAM_DOT_IDX tile (TaskKind 0/4; exec_task_block,
 * src/runtime/gpu_exec.cu:64-140, exec_task_cpu, src/runtime/kernels.h:
 * 1002-1258):  y[p*ystride + r] += dot(W[r], x + p*xstride), r < rows,
 * p < nx (0 means 1), W = w + (id_slot ? *id_slot * estride : 0) with the
 * id read ON THE DEVICE.  Validation as Graph::freeze
 * (src/runtime/graph.cpp:84-90): cols % block == 0, w_bytes == rows *
 * row_bytes, id_slot => estride != 0; and, since the columns run at
 * once, nx > 1 => ystride >= rows (overlapping outputs: FLH_ERR_ARG).
 * Alignment: x, y 4 bytes; w and estride 4 bytes for F32 / Q4_K, 2 bytes for
 * the 2-byte block formats (a row tile of rows 2 mod 4 bytes long).
 * fast = 0: canonical fp32 dequant-dot (fl_dot_row_any order, bitwise);
 * fast = 1: q8_K path for K formats whose bit is in i8k_mask, else q8_1
 * path for formats in i8_mask, else the "fast" fp32 dequant order
 * (dot_row_fast / dot_row_fast_q8_0 / dot_row_fast_dequant; F32 weights
 * always), exactly as exec_task_cpu.  cols = 0: every row's dot is 0.
 * int8 paths read the appendices written by flh_act_q8. */
int flh_stream_dot(int fmt, const void * w, uint64_t w_bytes, uint32_t rows,
                   uint32_t cols, const float * x, float * y, uint32_t nx,
                   uint32_t xstride, uint32_t ystride, const uint32_t * id_slot,
                   uint64_t estride, int fast, uint32_t i8_mask,
                   uint32_t i8k_mask, void * stream);

/* ACT_Q8 immediately followed by its STREAM_DOT consumer (the pair every
 * int8 tile of the reference graph builder emits, src/model/decoder.cpp:
 * 874-880,899-906), fused into one launch when the tile takes the q8_K path:
 * the kernel quantises x itself, workgroup 0 still writes both appendices,
 * and every output bit equals flh_act_q8 followed by flh_stream_dot (which is
 * what runs for any other format / mode).  No reference counterpart: the
 * reference always runs the two tasks separately. */
int flh_act_q8_stream_dot(int fmt, const void * w, uint64_t w_bytes, uint32_t rows,
                          uint32_t cols, float * x, float * y, uint32_t nx,
                          uint32_t xstride, uint32_t ystride,
                          const uint32_t * id_slot, uint64_t estride, int fast,
                          uint32_t i8_mask, uint32_t i8k_mask, void * stream);

/* RMSNORM of the column x (fl_op_rmsnorm, src/runtime/decode_params.h:101-106)
 * into xn -- fp32 y followed by its ACT_Q8 appendices, as flh_rmsnorm_act_q8
 * writes them with write_app = 1 -- then the single-column dot of it,
 * y[r] += dot(W[r], ACT_Q8(xn)) as flh_stream_dot: the decoder's
 * norm -> quant -> matvec chain (src/model/decoder.cpp:874-880; the tasks
 * RMSNORM, ACT_Q8, STREAM_DOT).  A Q4_K dot on the int8 path with at most
 * 8192 columns runs all three in one launch; anything else runs
 * flh_rmsnorm_act_q8 then flh_stream_dot.  The results are those of the two
 * calls, bit for bit.  x, wnorm and xn 16-byte aligned; xn must not overlap x. */
int flh_rmsnorm_stream_dot(int fmt, const void * w, uint64_t w_bytes, uint32_t rows,
                           uint32_t cols, const float * x, const float * wnorm, float eps,
                           float * xn, float * y, int fast, uint32_t i8_mask,
                           uint32_t i8k_mask, void * stream);

/* Execute a task table in array order on one stream (replaces the persistent
 * executor's per-task dispatch, exec_task_block, src/runtime/gpu_exec.cu:
 * 64-140, for a topologically ordered table such as run_serial walks,
 * src/runtime/graph.cpp:116-148).  Supported kinds: STREAM_DOT,
 * STREAM_DOT_IDX, ACT_Q8, MERGE, SIGNAL, RMSNORM, ROUTER_SEL, SILU_MUL,
 * WMERGE (an RMSNORM followed by the ACT_Q8 of its output is one
 * flh_rmsnorm_act_q8 launch, and with a single-column STREAM_DOT of that
 * activation after them, one flh_rmsnorm_stream_dot);
 * anything else -> FLH_ERR_UNSUPPORTED before any launch.  Consecutive
 * STREAM_DOT row tiles of one matrix (same fmt/cols/x/nx/strides, w and y
 * contiguous) are fused into one launch, and an ACT_Q8 followed by its
 * single-column q8_K consumer runs as flh_act_q8_stream_dot; results are
 * unchanged.  Masks are used as given, the same way as by every other entry
 * point (the same dot gives the same bits through any of them): pass the
 * reference's CPU masks (flh_default_masks) for the int8 parity path.  With
 * the reference's GPU defaults (kI8MaskGpuDefault / kI8KMaskGpuDefault,
 * src/runtime/kernels.h:927-940) Q6_K takes the fp32 dequant route (the
 * same order on one wave per row, about 2x the int8 route's time at the
 * vocab head); with the CPU masks IQ2_XXS / IQ3_XXS take it.
 * The param blocks that RMSNORM, ROUTER_SEL, SILU_MUL and WMERGE tasks point
 * to through aux are read by the host when the table is issued, so they must
 * be host-readable (host, pinned or managed memory; flh_host_alloc gives
 * pinned memory): a block in device memory is rejected with FLH_ERR_ARG
 * before anything is launched.  The buffers those blocks name, and every
 * other Task pointer, are device memory. */
int flh_exec_tasks(const flh_task * tasks, uint32_t n, int fast,
                   uint32_t i8_mask, uint32_t i8k_mask, void * stream);

/* Bit-exact dequantisation of whole rows to fp32, out[r*cols + c]
 * (dequant_chunk, src/runtime/kernels.h:162-242). */
int flh_dequant(int fmt, const void * w, uint32_t rows, uint32_t cols,
                float * out, void * stream);

/* ------------------------------------------------------------------ MoE -- */
/* Grouped expert matvec (the STREAM_DOT_IDX expert tiles of
 * src/model/decoder.cpp:941-996, grouped by expert): for every routed pair
 * i = tok*top_k + slot with e = ids[i],
 *   y[i*ystride + r] += dot(W_e[r], x + xi*xstride),  W_e = w + e*estride,
 * xi = tok (x_per_slot = 0) or i (x_per_slot = 1).  Each expert's weights
 * are streamed once for all of its pairs (Q4_K, Q6_K: the q8_K int8 path);
 * Q8_0, Q5_0, IQ2_XXS and IQ3_XXS run the q8_1 int8 path one pair at a time,
 * as the reference's per-pair tiles do: one routed launch where its plan
 * holds the shape (16-byte aligned w, x and estride, at most ~14.5K columns;
 * IQ: a multiple of 2048), else one STREAM_DOT_IDX tile per pair (up to 16384
 * columns; the ids must then be < n_expert, as ROUTER_SEL writes them).
 * cols a positive multiple of 256 (0 is FLH_ERR_ARG).  Every output is bitwise equal to the per-pair
 * STREAM_DOT_IDX tile. */
int flh_moe_dot(int fmt, const void * w, uint64_t estride, uint32_t rows,
                uint32_t cols, const uint32_t * ids, uint32_t ntok,
                uint32_t top_k, uint32_t n_expert, const float * x,
                uint32_t xstride, uint32_t x_per_slot, float * y,
                uint32_t ystride, void * stream);

/* ROUTER_SEL for ntok tokens (fl_op_router_sel, decode_params.h:234-265):
 * logits [ntok][n_expert], ids/gates [ntok][top_k]. */
int flh_router_sel(const float * logits, uint32_t ntok, uint32_t n_expert,
                   uint32_t top_k, uint32_t norm, float scale, uint32_t * ids,
                   float * gates, void * stream);
/* ROUTER_SEL followed by the grouped expert matvec of its routing, as one
 * launch where the grouped kernels take it (n_expert <= 64, top_k <= 8,
 * ntok*top_k <= 256; otherwise two): every workgroup routes the ntok tokens
 * itself with the same float operations as flh_router_sel, one of them
 * writes ids and gates.  Outputs (ids, gates, y) equal flh_router_sel then
 * flh_moe_dot bit for bit.  Replaces the ROUTER_SEL task
 * (src/runtime/decode_params.h:234-265) and the STREAM_DOT_IDX expert tiles
 * it feeds (src/model/decoder.cpp:941-996) for one MoE layer. */
int flh_router_moe_dot(int fmt, const void * w, uint64_t estride, uint32_t rows,
                       uint32_t cols, const float * logits, uint32_t ntok,
                       uint32_t n_expert, uint32_t top_k, uint32_t norm, float scale,
                       uint32_t * ids, float * gates, const float * x, uint32_t xstride,
                       uint32_t x_per_slot, float * y, uint32_t ystride, void * stream);
/* SILU_MUL over ncol columns (fl_op_silu_mul, decode_params.h:267-272):
 * h[c*hstride + i] = silu(g[c*gstride + i]) * u[c*gstride + i]. */
int flh_silu_mul(const float * gate, const float * up, float * h, uint32_t n,
                 uint32_t ncol, uint32_t gstride, uint32_t hstride, void * stream);
/* SILU_MUL over ncol columns followed by ACT_Q8 of each h column, in one
 * launch: h holds ACT_Q8 buffers (fp32 h, then its q8_1 and q8_K appendices,
 * columns hstride floats apart, 16-byte aligned); the bytes written equal
 * flh_silu_mul followed by flh_act_q8 (fl_op_silu_mul then fl_exec_act_q8,
 * decode_params.h:267-272, quants.h:404-416; the decoder's down-projection
 * input, decoder.cpp:874-880).  flh_exec_tasks fuses such a task pair itself. */
int flh_silu_mul_act_q8(const float * gate, const float * up, float * h, uint32_t n,
                        uint32_t ncol, uint32_t gstride, uint32_t hstride, void * stream);
/* RMSNORM of one column (fl_op_rmsnorm, decode_params.h:101-106:
 * y = (x * s) * wnorm, s = 1 / sqrtf(mean(x^2) + eps)) with, when write_app,
 * the ACT_Q8 of y in the same launch (y is then an ACT_Q8 buffer, 16-byte
 * aligned, and its appendices get the bytes flh_act_q8 would write from
 * these y values: the decoder's norm -> quant chain, decoder.cpp:874-880).
 * The reference (CPU-only op) sums the squares strictly in order; here the
 * 16 waves of one workgroup sum them as a tree (lane partials over its
 * elements in order, wave and workgroup trees in a fixed order), so s
 * and y agree with the reference to float rounding, not bit for bit (the
 * tests bound it); everything after s is the reference's arithmetic. */
int flh_rmsnorm_act_q8(const float * x, const float * wnorm, float * y, uint32_t n, float eps,
                       int write_app, void * stream);
/* WMERGE over ncol columns (fl_op_wmerge, decode_params.h:274-295): column c
 * reads parts + c*pstride ([n_parts][n]), gates + c*n_parts, add1/add2 +
 * c*ystride, writes y + c*ystride. */
int flh_wmerge(const float * parts, const float * gates, const float * add1,
               const float * add2, float * y, float scale, uint32_t n_parts,
               uint32_t n, uint32_t n_full, uint32_t ncol, uint32_t pstride,
               uint32_t ystride, void * stream);

/* ---------------------------------------------------------------- GGUF -- */
/* GGUF v2/v3 reader (replaces fastllm::Gguf, src/model/gguf.h:28-79,
 * src/model/gguf.cpp:133-303).  The file is mmapped read-only; metadata and
 * tensor infos are parsed at open.  Split models named
 * "<stem>-NNNNN-of-MMMMM.gguf" map every shard: metadata comes from the shard
 * named, tensors are merged in shard order, each with offsets relative to its
 * own shard's data section; split.tensors.count, when present, must equal the
 * tensors mapped.  Where Gguf::open aborts (bad magic / version / KV type /
 * n_dims, truncation) this returns FLH_ERR_FORMAT; a missing file or shard
 * gives FLH_ERR_IO (Gguf::open returns false).  Stricter than the reference:
 * a tensor payload past the end of its file, an array of an unsized element
 * type and a general.alignment that is not a power of two are FLH_ERR_FORMAT.
 * Host-only: nothing before flh_gguf_upload* touches the GPU. */
typedef struct flh_gguf flh_gguf;

/* One tensor info (GgufTensor, src/model/gguf.h:19-27).  Pointers stay valid
 * until flh_gguf_close. */
typedef struct flh_gguf_tensor {
    const char * name;
    size_t name_len;
    uint32_t type;             /* ggml_type id */
    int32_t fmt;               /* FLH_FMT_* (Gguf::fmt_of), -1 if none */
    int32_t n_dims;
    uint64_t ne[4];            /* unused dims are 1 */
    uint64_t offset;           /* relative to its shard's data section */
    uint64_t nbytes;           /* payload bytes; 0 for types with no size */
    int32_t shard;
    const void * data;         /* host pointer into the mapping (Gguf::data) */
} flh_gguf_tensor;

/* A STREAM_DOT weight bound from a tensor (DecoderImpl::load_tensor,
 * src/model/decoder.cpp:186-206): cols = ne[0], rows = ne[1], nexp = ne[2]
 * for 3-D expert stacks (else 1), estride = rows*row_bytes when nexp > 1. */
typedef struct flh_weight {
    int32_t fmt;
    uint32_t rows, cols, nexp;
    uint64_t row_bytes, w_bytes, estride;
    const void * host;         /* mapping pointer of expert 0 */
    uint64_t tensor;           /* tensor index */
} flh_weight;

int flh_gguf_open(const char * path, flh_gguf ** out);
int flh_gguf_close(flh_gguf * g);
uint32_t flh_gguf_alignment(const flh_gguf * g);   /* of the named shard */
int flh_gguf_n_shards(const flh_gguf * g);
uint64_t flh_gguf_n_tensors(const flh_gguf * g);
int flh_gguf_tensor_info(const flh_gguf * g, uint64_t i, flh_gguf_tensor * out);
/* index of the first tensor of that name (Gguf::find), -1 if none */
int64_t flh_gguf_find(const flh_gguf * g, const char * name);
/* Gguf::fmt_of / Gguf::type_name (src/model/gguf.cpp:82-109) */
int flh_gguf_fmt_of(uint32_t ggml_type);
const char * flh_gguf_type_name(uint32_t ggml_type);
/* Metadata (Gguf::has / kv_i / kv_f / kv_s / kv_sarr, gguf.cpp:267-293):
 * integer kinds and bool read as int64, f32/f64 as double, each readable
 * through the other getter; strings and string arrays verbatim (len
 * receives the byte length, strings may hold NUL bytes).  Arrays of other
 * element types are skipped.  kv_sarr_len is -1 for an absent key. */
int flh_gguf_has(const flh_gguf * g, const char * key);
int64_t flh_gguf_kv_i(const flh_gguf * g, const char * key, int64_t dflt);
double flh_gguf_kv_f(const flh_gguf * g, const char * key, double dflt);
const char * flh_gguf_kv_s(const flh_gguf * g, const char * key, const char * dflt,
                           size_t * len);
int64_t flh_gguf_kv_sarr_len(const flh_gguf * g, const char * key);
const char * flh_gguf_kv_sarr_at(const flh_gguf * g, const char * key, uint64_t i,
                                 size_t * len);
/* FLH_ERR_ARG for a missing tensor, FLH_ERR_UNSUPPORTED for a type with no
 * Fmt (the two failures of load_tensor). */
int flh_gguf_weight(const flh_gguf * g, const char * name, flh_weight * out);

/* Host -> device.  The reference reads the mapping in place through unified
 * memory (decoder.cpp:203); here weights are copied into HBM once.  Bytes go
 * through a ring of pinned staging buffers filled by host threads while the
 * DMA engine drains the previous one; both calls return when every byte is
 * on the device.  flh_gguf_upload copies tensor i to dst (dst_bytes >=
 * nbytes).  flh_gguf_upload_all allocates, per shard, one 256-B aligned arena
 * block for the span of its tensor payloads and copies that span as-is, so
 * dev_ptrs[i] (n_tensors entries) = block + offset keeps the file's alignment;
 * dev_ptrs[i] = NULL where nbytes = 0.  Uploads from several threads are
 * serialised. */
int flh_gguf_upload(const flh_gguf * g, uint64_t i, void * dst, uint64_t dst_bytes,
                    void * stream);
int flh_gguf_upload_all(const flh_gguf * g, flh_arena * arena, void ** dev_ptrs,
                        void * stream);

/* ----------------------------------------------------- synthetic inputs -- */
/* dst[i] = mean + stddev * N(0,1) from a counter-based generator keyed by
 * (seed, i); a fraction outlier_frac of entries is multiplied by
 * outlier_scale.  Deterministic for a given (seed, n). */
int flh_fill_normal(float * dst, size_t n, uint64_t seed, float mean,
                    float stddev, float outlier_frac, float outlier_scale,
                    void * stream);
/* fp32 rows -> Q8_0 / Q4_K / Q6_K blocks on the device; flh_quantize_host
 * produces the same bytes on the host.  (The reference ships no weight
 * quantizer; these are this backend's own, for synthetic weights.) */
int flh_quantize(int fmt, const float * src, uint32_t rows, uint32_t cols,
                 void * dst, void * stream);
int flh_quantize_host(int fmt, const float * src, uint32_t rows, uint32_t cols,
                      void * dst);

#ifdef __cplusplus
}
#endif
#endif /* FASTLLM_HIP_H */
