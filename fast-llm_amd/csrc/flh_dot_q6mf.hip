// flh_dot_q6mf.hip -- several-column Q6_K x q8_K row-dots on gfx950's int8
// matrix cores (speculative verify of Q6_K matrices, e.g. a vocab head).
//
// fl_dot_i8k_q6_K (src/runtime/quants.h:563-594) per row and column:
//   iacc_sb = sum_i sc_i * (idot_i - 32 bsum_i),  i = the 16 sub-blocks of 16
//   a[sb & 3] = fmaf(d * dk, (float)iacc_sb, a[sb & 3]);  y += (a0 + a1) + (a2 + a3)
// with idot_i over the unsigned 6-bit values.  Here sum_e (q_e - 32) x_e is
// the same integer as idot_i - 32 bsum_i, and q - 32 fits int8, so each
// sub-block's dot is one v_mfma_i32_32x32x16_i8 over a 32-row tile:
//   D[n][r] = sum_k x_n[16 i + k] * (q_r[16 i + k] - 32)
// (A = activation columns n, zero for n >= nx; B = the tile's 32 weight rows).
// Lane l supplies row r = l % 32 and k-half h = l / 32 (8 elements of each
// sub-block) and receives D for row r and columns 4h .. 4h + 3, so the scale
// products and the reference's float fold run per lane, in superblock order,
// on registers: bitwise equal to the reference for every column.
//
// Weights stream HBM -> LDS with direct-to-LDS 16-byte loads, one superblock
// of the tile per ring stage (32 rows x 15 aligned segments; a row's 210
// bytes start 2-byte aligned, so the lane reads aligned dwords and realigns);
// each wave owns its ring and runs its own 32-row tiles.  The activation
// columns' q8_K blocks are staged once per workgroup.  With fewer tiles than
// waves on the chip (SPLIT), four waves share a tile: wave j streams the
// superblocks sb = j mod 4, which are exactly the reference's chain a[j], and
// wave 0 of the four adds the four chains through LDS in the reference's
// (a0 + a1) + (a2 + a3), so the bits are the same either way.
#include "flh_kstream.h"
#include "flh_internal.h"
#include "flh_status.h"

namespace flh {

typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr uint32_t Q6MF_SLOT = 7680;       // ring stage: 32 rows x 15 segments
constexpr uint32_t Q6MF_W = 8;             // waves per workgroup
constexpr uint32_t Q6MF_RSTRIDE = 240;     // LDS bytes per row in a stage
constexpr uint32_t Q6MF_ZERO = 272;        // zero bytes the A reads of columns >= NC use

__host__ __device__ inline uint32_t q6mf_xqs(uint32_t nsb) { return 256 * nsb + 16; }
__host__ __device__ inline size_t q6mf_smem(uint32_t NC, uint32_t D, uint32_t nsb, uint32_t W) {
    return (size_t)W * D * Q6MF_SLOT + (size_t)NC * q6mf_xqs(nsb) + Q6MF_ZERO + (size_t)4 * (NC < 8 ? 8 : NC) * nsb;
}

// The lane's 12 runs of 8 bytes (ql: 64hh + 32a + 16b + 8h, qh: 128 + 32hh +
// 16b + 8h) as 3 aligned dwords each, from base = the run origin rounded down
// to 4 bytes; and the 24 bytes from the scales' aligned origin.
__device__ __forceinline__ void q6mf_ld_runs(uint32_t base, uint32_t sbase, u32x2v (&R)[18], u32x2v (&S)[3]) {
    asm volatile(
        "ds_read2_b32 %0, %21 offset0:0 offset1:1\n\tds_read2_b32 %1, %21 offset0:4 offset1:5\n\t"
        "ds_read2_b32 %2, %21 offset0:8 offset1:9\n\tds_read2_b32 %3, %21 offset0:12 offset1:13\n\t"
        "ds_read2_b32 %4, %21 offset0:16 offset1:17\n\tds_read2_b32 %5, %21 offset0:20 offset1:21\n\t"
        "ds_read2_b32 %6, %21 offset0:24 offset1:25\n\tds_read2_b32 %7, %21 offset0:28 offset1:29\n\t"
        "ds_read2_b32 %8, %21 offset0:32 offset1:33\n\tds_read2_b32 %9, %21 offset0:36 offset1:37\n\t"
        "ds_read2_b32 %10, %21 offset0:40 offset1:41\n\tds_read2_b32 %11, %21 offset0:44 offset1:45\n\t"
        "ds_read2_b32 %12, %21 offset0:2 offset1:6\n\tds_read2_b32 %13, %21 offset0:10 offset1:14\n\t"
        "ds_read2_b32 %14, %21 offset0:18 offset1:22\n\tds_read2_b32 %15, %21 offset0:26 offset1:30\n\t"
        "ds_read2_b32 %16, %21 offset0:34 offset1:38\n\tds_read2_b32 %17, %21 offset0:42 offset1:46\n\t"
        "ds_read2_b32 %18, %22 offset0:0 offset1:1\n\tds_read2_b32 %19, %22 offset0:2 offset1:3\n\t"
        "ds_read2_b32 %20, %22 offset0:4 offset1:5\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(R[0]), "=&v"(R[1]), "=&v"(R[2]), "=&v"(R[3]), "=&v"(R[4]), "=&v"(R[5]), "=&v"(R[6]),
          "=&v"(R[7]), "=&v"(R[8]), "=&v"(R[9]), "=&v"(R[10]), "=&v"(R[11]), "=&v"(R[12]), "=&v"(R[13]),
          "=&v"(R[14]), "=&v"(R[15]), "=&v"(R[16]), "=&v"(R[17]), "=&v"(S[0]), "=&v"(S[1]), "=&v"(S[2])
        : "v"(base), "v"(sbase) : "memory");
}
// the 16 A operands of a superblock (8 bytes at 16 i from base) and the
// four dk of the lane's columns
__device__ __forceinline__ void q6mf_ld_x(uint32_t base, uint32_t dbase, u32x2v (&A)[16], u32x4a & dk) {
    asm volatile(
        "ds_read_b64 %0, %17\n\tds_read_b64 %1, %17 offset:16\n\tds_read_b64 %2, %17 offset:32\n\t"
        "ds_read_b64 %3, %17 offset:48\n\tds_read_b64 %4, %17 offset:64\n\tds_read_b64 %5, %17 offset:80\n\t"
        "ds_read_b64 %6, %17 offset:96\n\tds_read_b64 %7, %17 offset:112\n\tds_read_b64 %8, %17 offset:128\n\t"
        "ds_read_b64 %9, %17 offset:144\n\tds_read_b64 %10, %17 offset:160\n\tds_read_b64 %11, %17 offset:176\n\t"
        "ds_read_b64 %12, %17 offset:192\n\tds_read_b64 %13, %17 offset:208\n\tds_read_b64 %14, %17 offset:224\n\t"
        "ds_read_b64 %15, %17 offset:240\n\tds_read_b128 %16, %18\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(A[0]), "=&v"(A[1]), "=&v"(A[2]), "=&v"(A[3]), "=&v"(A[4]), "=&v"(A[5]), "=&v"(A[6]),
          "=&v"(A[7]), "=&v"(A[8]), "=&v"(A[9]), "=&v"(A[10]), "=&v"(A[11]), "=&v"(A[12]), "=&v"(A[13]),
          "=&v"(A[14]), "=&v"(A[15]), "=&v"(dk)
        : "v"(base), "v"(dbase) : "memory");
}

template <int NC, int D, bool SPLIT, int NW>
__global__ __launch_bounds__(64 * NW) void k_dot_q6mf(DotArgs a, uint32_t nwt) {
    static_assert(NC == 4 || NC == 8 || NC == 16, "column capacity");
    static_assert(!SPLIT || (NC <= 8 && NW % 4 == 0), "a split workgroup holds whole quads");
    constexpr int NCX = NC < 8 ? 8 : NC;                          // dk slots per superblock
    constexpr int NCL = NC == 16 ? 8 : 4;                          // columns per lane
    extern __shared__ __attribute__((aligned(16))) uint8_t q6_sm[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t cols = a.cols, nsb = cols >> 8, rows = a.rows, nx = a.nx;
    const uint32_t RB = nsb * 210, XQS = q6mf_xqs(nsb);
    uint8_t * ring = q6_sm + (size_t)wave * D * Q6MF_SLOT;
    uint8_t * xq = q6_sm + (size_t)NW * D * Q6MF_SLOT;
    uint8_t * zr = xq + (size_t)NC * XQS;
    float * xd = reinterpret_cast<float *>(zr + Q6MF_ZERO);       // [nsb][NCX]
    const uint8_t * w = a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0);

    // activations: the NC columns' int8 values (zero for columns >= nx), dk
    {
        const uint32_t per = nsb * 64;                            // dwords of a column
        for (uint32_t i = tid; i < NC * per; i += 64 * NW) {
            const uint32_t n = i / per, q = i - n * per, sb = q >> 6, j = q & 63;
            uint32_t v = 0;
            if (n < nx) {
                const uint8_t * app = reinterpret_cast<const uint8_t *>(a.x + (size_t)n * a.xstride) + xqk_off(cols);
                v = *reinterpret_cast<const uint32_t *>(app + 292 * (size_t)sb + 36 + 4 * j);   // {d, bsums[16], qs[256]}
            }
            *reinterpret_cast<uint32_t *>(xq + (size_t)n * XQS + 256 * sb + 4 * j) = v;
        }
        for (uint32_t i = tid; i < Q6MF_ZERO / 4; i += 64 * NW) reinterpret_cast<uint32_t *>(zr)[i] = 0;
        for (uint32_t i = tid; i < nsb * NCX; i += 64 * NW) {
            const uint32_t sb = i / NCX, n = i % NCX;
            float v = 0.f;
            if (n < nx) {
                const uint8_t * app = reinterpret_cast<const uint8_t *>(a.x + (size_t)n * a.xstride) + xqk_off(cols);
                v = *reinterpret_cast<const float *>(app + 292 * (size_t)sb);
            }
            xd[i] = v;
        }
        __syncthreads();
    }

    const uint32_t T = (rows + 31) / 32;
    // tiles: a wave (SPLIT: a quad of waves) takes tiles tb, tb + tstride, ...;
    // a split wave j streams superblocks j, j + 4, ... of its quad's tile
    const uint32_t j4 = SPLIT ? (wave & 3) : 0;
    const uint32_t tb = SPLIT ? blockIdx.x * (NW / 4) + (wave >> 2) : blockIdx.x * NW + wave;
    const uint32_t tstride = SPLIT ? nwt / 4 : nwt;
    const uint32_t sb0 = j4, sstep = SPLIT ? 4 : 1;
    const uint32_t cnt = SPLIT ? (j4 < nsb ? (nsb - 1 - j4) / 4 + 1 : 0) : nsb;   // superblocks per tile
    const uint32_t ntw = tb < T ? (T - tb + tstride - 1) / tstride : 0;   // tiles of this wave (uniform)
    const uint32_t NI = ntw * cnt;
    // DMA of item (tile k of this wave, superblock sb) into stage st: position
    // p = 64 j + lane holds segment p % 15 of row p / 15 (p < 480).  A row's
    // 210 bytes start 2-byte aligned, so from the 16-byte boundary below them
    // they span at most 14 segments (offset <= 14, 14 + 210 <= 224): segment 14
    // repeats segment 13, and no segment reads past the 16-byte granule that
    // holds the superblock's last byte.  Per lane the row and the segment
    // offset of each j are fixed; per item only the tile's row limit moves.
    uint32_t prow[8], pseg[8];
#pragma unroll
    for (uint32_t jj = 0; jj < 8; ++jj) {
        const uint32_t p = 64 * jj + lane;
        prow[jj] = p < 480 ? p / 15 : 31;
        pseg[jj] = p < 480 ? 16 * min(p % 15, 13u) : 0;
    }
    auto issue = [&](uint32_t k, uint32_t c, uint32_t st) __attribute__((always_inline)) {
        const uint32_t r0 = (tb + k * tstride) * 32, lim = rows - 1 - r0;   // r0 < rows: tile k exists
        const uint32_t sb = sb0 + sstep * c;
        const uintptr_t base = (uintptr_t)(w + (size_t)r0 * RB + 210 * (size_t)sb);
        uint8_t * dst = ring + (size_t)st * Q6MF_SLOT;
#pragma unroll
        for (uint32_t jj = 0; jj < 8; ++jj) {
            const uintptr_t a0 = (base + __umul24(min(prow[jj], lim), RB)) & ~(uintptr_t)15;
            if (jj < 7 || lane < 32)                              // positions 480..511 are not in the stage
                __builtin_amdgcn_global_load_lds(GPTR(a0 + pseg[jj]), LPTR(dst + 1024 * jj), 16, 0, 0);
        }
    };
    uint32_t fk = 0, fc = 0;                                      // next item to issue
    auto issue_next = [&](uint32_t st) __attribute__((always_inline)) {
        issue(fk < ntw ? fk : ntw - 1, fk < ntw ? fc : 0, st);
        if (++fc == cnt) { fc = 0; ++fk; }
    };
    if (!SPLIT && NI == 0) return;                                // no tile: nothing to stream
    if (NI != 0) {
#pragma unroll
        for (int d = 0; d + 1 < D; ++d) issue_next((uint32_t)d);
    }

    const uint32_t r = lane & 31, h = lane >> 5;
    f4v a4[NCL];                                                 // [column][accumulator]
    int iacc[NCL];
    uint32_t it = 0;
    auto item = [&](uint32_t k, uint32_t c) __attribute__((always_inline)) {
    const uint32_t st = it % D;
    issue_next((it + D - 1) % D);
    WAIT_VM(8 * (D - 1));
    const uint32_t sb = sb0 + sstep * c;
    const uint32_t r0 = (tb + k * tstride) * 32, ra = min(r0 + r, rows - 1);
    const uintptr_t A = (uintptr_t)(w + (size_t)ra * RB + 210 * (size_t)sb);
    const uint32_t sh = (uint32_t)(A & 15);
    const uint32_t rbase = lds_off(ring + (size_t)st * Q6MF_SLOT) + Q6MF_RSTRIDE * r + (sh & ~3u);
    u32x2v R[18], S3[3];
    q6mf_ld_runs(rbase + 8 * h, rbase + 192, R, S3);
    u32x2v X[16];
    u32x4a dk;
    const uint32_t n = lane & 31;
    const uint32_t xbase = n < NC ? lds_off(xq) + n * XQS + 256 * sb + 8 * h : lds_off(zr);
    q6mf_ld_x(xbase, lds_off(xd) + 4 * NCX * sb + 16 * h, X, dk);
    u32x4a dk2 = dk;
    if constexpr (NC == 16) dk2 = *reinterpret_cast<const u32x4a *>(xd + NCX * sb + 8 + 4 * h);   // columns 8 + 4h ..
    const uint32_t s8 = 8 * (sh & 3);
    uint32_t W[12][2];
#pragma unroll
    for (int q = 0; q < 12; ++q) {
        const uint32_t d2 = (q & 1) ? R[12 + (q >> 1)].y : R[12 + (q >> 1)].x;
        W[q][0] = __builtin_amdgcn_alignbyte(R[q].y, R[q].x, s8 >> 3);
        W[q][1] = __builtin_amdgcn_alignbyte(d2, R[q].y, s8 >> 3);
    }
    const uint32_t s0 = S3[0].x, s1 = S3[0].y, s2 = S3[1].x, s3 = S3[1].y, s4 = S3[2].x, s5 = S3[2].y;
    const uint32_t SC[4] = {__builtin_amdgcn_alignbyte(s1, s0, s8 >> 3), __builtin_amdgcn_alignbyte(s2, s1, s8 >> 3),
                            __builtin_amdgcn_alignbyte(s3, s2, s8 >> 3), __builtin_amdgcn_alignbyte(s4, s3, s8 >> 3)};
    const float dw = h2f(__builtin_amdgcn_alignbyte(s5, s4, s8 >> 3) & 0xFFFFu);
#pragma unroll
    for (int v = 0; v < NCL; ++v) iacc[v] = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int hh = i >> 3, s4i = (i >> 1) & 3, b = i & 1;
        const int q = 4 * hh + 2 * (s4i & 1) + b, qq = 8 + 2 * hh + b;
        uint32_t Bv[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t qlw = W[q][t], qhw = W[qq][t];
            const uint32_t nib = s4i < 2 ? (qlw & 0x0F0F0F0Fu) : ((qlw >> 4) & 0x0F0F0F0Fu);
            const uint32_t hb = ((qhw >> (2 * s4i)) & 0x03030303u) << 4;
            Bv[t] = ((nib | hb) + 0x60606060u) ^ 0x80808080u;  // q - 32 per byte
        }
        const long av = (long)(((uint64_t)X[i].y << 32) | X[i].x);
        const long bv = (long)(((uint64_t)Bv[1] << 32) | Bv[0]);
        const v16i c = {};
        const v16i dd = __builtin_amdgcn_mfma_i32_32x32x16_i8(av, bv, c, 0, 0, 0);
        const int sc = (int)(int8_t)((SC[i >> 2] >> (8 * (i & 3))) & 0xFFu);
#pragma unroll
        for (int v = 0; v < NCL; ++v) iacc[v] += __mul24(sc, dd[v]);   // D row 4h + v (v < 4), 8 + 4h + v - 4
        if (i & 1) __builtin_amdgcn_sched_barrier(0);        // two sub-blocks' results live at a time
    }
    // the reference fold: a[sb & 3] = fmaf(d * dk, (float)iacc, a[sb & 3])
    const float dkv[8] = {__uint_as_float(dk.x), __uint_as_float(dk.y), __uint_as_float(dk.z), __uint_as_float(dk.w),
                          __uint_as_float(dk2.x), __uint_as_float(dk2.y), __uint_as_float(dk2.z), __uint_as_float(dk2.w)};
    const uint32_t q3 = SPLIT ? 0 : (sb & 3);            // a split wave runs the chain sb & 3 alone
#pragma unroll
    for (int v = 0; v < NCL; ++v) {
        const float m = dw * dkv[v], f = (float)iacc[v];
        if (q3 == 0) a4[v][0] = fmaf(m, f, a4[v][0]);              // uniform branches: a4 stays in registers
        else if (q3 == 1) a4[v][1] = fmaf(m, f, a4[v][1]);
        else if (q3 == 2) a4[v][2] = fmaf(m, f, a4[v][2]);
        else a4[v][3] = fmaf(m, f, a4[v][3]);
    }
        ++it;
    };
    auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int v = 0; v < NCL; ++v)
#pragma unroll
            for (int q = 0; q < 4; ++q) a4[v][q] = 0.f;
    };
    // y += (a0 + a1) + (a2 + a3) for the lane's row of tile k and its columns
    auto store = [&](uint32_t k) __attribute__((always_inline)) {
        const uint32_t r0 = (tb + k * tstride) * 32;
        const uint32_t rr = r0 + r;
        if (rr < rows) {
#pragma unroll
            for (int v = 0; v < NCL; ++v) {
                const uint32_t col = 4 * h + v + (v >= 4 ? 4 : 0);
                if (col < nx) {
                    float * y = a.y + (size_t)col * a.ystride + rr;
                    *y = *y + ((a4[v][0] + a4[v][1]) + (a4[v][2] + a4[v][3]));
                }
            }
        }
    };
    if constexpr (!SPLIT) {
        uint32_t k = 0, c = 0;
        for (uint32_t i = 0; i < NI; ++i) {
            if (c == 0) zero_acc();
            item(k, c);
            if (++c == cnt) {                                     // the tile's rows are done
                store(k);
                c = 0;
                ++k;
            }
        }
    } else {
        // every wave of the workgroup runs the same rounds (barriers); the
        // quad's waves 1-3 leave their chain (4 floats per lane) in the ring
        // stage their last item used, which their next DMA waits for the
        // second barrier to overwrite, and wave 0 of the quad folds them in
        const uint32_t R = (T + tstride - 1) / tstride;
        uint8_t * quad = q6_sm + (size_t)(wave & ~3u) * D * Q6MF_SLOT;
        for (uint32_t k = 0; k < R; ++k) {
            zero_acc();
            const bool live = k < ntw;
            if (live)
                for (uint32_t c = 0; c < cnt; ++c) item(k, c);
            if (live && j4 != 0 && cnt != 0) {
                float4 * pp = reinterpret_cast<float4 *>(ring + (size_t)((it - 1) % D) * Q6MF_SLOT) + lane;
                *pp = make_float4(a4[0][0], a4[1][0], a4[2][0], a4[3][0]);
            }
            __syncthreads();
            if (live && j4 == 0) {
#pragma unroll
                for (uint32_t jw = 1; jw < 4; ++jw) {
                    const uint32_t cw = jw < nsb ? (nsb - 1 - jw) / 4 + 1 : 0;
                    if (cw != 0) {
                        const uint32_t stw = ((k + 1) * cw - 1) % D;
                        const float4 pv = *(reinterpret_cast<const float4 *>(quad + ((size_t)jw * D + stw) * Q6MF_SLOT) + lane);
                        a4[0][jw] = pv.x; a4[1][jw] = pv.y; a4[2][jw] = pv.z; a4[3][jw] = pv.w;
                    }
                }
                store(k);
            }
            __syncthreads();
        }
    }
    WAIT_VM(0);                                                   // the spare DMAs of the last items
}

// 2..16 Q6_K columns with cols a multiple of 256; FLH_ERR_UNSUPPORTED (nothing
// launched) when the shape does not fit the LDS plan.
int launch_dot_q6mf(const DotArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    if (nsb == 0 || nsb * 210ull >= (1u << 24) || (a.cols & 255) || a.nx < 2 || a.nx > 16 || ((uintptr_t)a.x & 3) ||
        ((uintptr_t)a.w & 1) || (a.estride & 1))
        return FLH_ERR_UNSUPPORTED;
    if (a.rows == 0) return FLH_OK;
    const uint32_t NC = a.nx <= 4 ? 4 : a.nx <= 8 ? 8 : 16;
    // 16 columns: 6 waves, so the ring and the 16 columns' activations fit
    const uint32_t W = NC == 16 ? 6 : Q6MF_W;
    // the deepest ring that fits: 3 superblocks in flight per wave where possible
    const int D = q6mf_smem(NC, 3, nsb, W) <= lds_limit() ? 3 : 2;
    const size_t smb = q6mf_smem(NC, D, nsb, W);
    if (smb > lds_limit()) return FLH_ERR_UNSUPPORTED;
    const uint32_t T = (a.rows + 31) / 32;
    // fewer tiles than waves on the chip: a quad of waves shares each tile,
    // one wave per accumulator chain sb & 3 (up to 8 columns)
    const bool split = T < (uint32_t)num_cus() * W;
    if (split && NC == 16) return FLH_ERR_UNSUPPORTED;
    const uint32_t per = split ? W / 4 : W;                       // tiles in flight per workgroup
    uint32_t G = (uint32_t)num_cus();
    if (G > (T + per - 1) / per) G = (T + per - 1) / per;
    const uint32_t nwt = G * W;
    auto go = [&](auto kern) {
        if (int rc = lds_fits((const void *)kern, smb, "k_dot_q6mf: LDS over the limit")) return rc;
        (void)hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smb);
        hipLaunchKernelGGL(kern, dim3(G), dim3(64 * W), smb, s, a, nwt);
        return hip_check(hipGetLastError(), "k_dot_q6mf launch");
    };
    constexpr int W8 = (int)Q6MF_W;
    if (NC == 16) return D == 3 ? go(k_dot_q6mf<16, 3, false, 6>) : go(k_dot_q6mf<16, 2, false, 6>);
    if (split) {
        if (NC == 4) return D == 3 ? go(k_dot_q6mf<4, 3, true, W8>) : go(k_dot_q6mf<4, 2, true, W8>);
        return D == 3 ? go(k_dot_q6mf<8, 3, true, W8>) : go(k_dot_q6mf<8, 2, true, W8>);
    }
    if (NC == 4) return D == 3 ? go(k_dot_q6mf<4, 3, false, W8>) : go(k_dot_q6mf<4, 2, false, W8>);
    return D == 3 ? go(k_dot_q6mf<8, 3, false, W8>) : go(k_dot_q6mf<8, 2, false, W8>);
}

}  // namespace flh
