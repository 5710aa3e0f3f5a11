// flh_dot_mfma.hip -- multi-column Q4_K x q8_K row-dots (speculative verify,
// grouped MoE experts) on gfx950's int8 matrix cores.
//
// With several activation columns the per-lane VALU dot of the streaming
// kernel (flh_dot_kstream.hip) becomes instruction-bound (about 300 wave
// instructions per 2304-byte chunk at 4 columns).  Here the integer dot of
// every 32-weight sub-block is one MFMA over a 16-row tile:
//
//   D[n][r] = sum_k x_n[k] * q_r[k]      v_mfma_i32_16x16x32_i8
//             A = activations (16 columns x 32), B = weight nibbles (32 x 16 rows)
//
// so lane l owns weight row r = l % 16 and activation columns 4*(l/16) + i,
// and decodes only its own row's 6-bit scales.  The scale-weighted sum
// iacc = sum_g sc_g * D_g is exact integer VALU work.  With 4 or 8 columns
// the A operand is block-diagonal instead (the column block of A rows 4g..
// (resp. 8h..) sees only k-slice g (resp. 2h, 2h + 1), and lane row g's B
// slice carries its own sub-blocks), so no output row is idle: a lane holds
// whole sub-block dots of 2 (resp. 4) sub-blocks and iacc is 8 (resp. 16)
// products plus an exact cross-lane integer sum (permlane swaps).  The min term
// imins = sum_g m_g * (bsum[2g] + bsum[2g+1]) is a 16x16x8 product done as two
// v_mfma_f32_16x16x4f32 whose operands and sums are integers below 2^24, so
// it is exact too.  The (row, column, superblock) integer terms are parked in
// LDS and folded in the reference order (acc[sb & 3], fl_dot_i8k_q4_K,
// src/runtime/quants.h:538-561), so every output is bitwise equal to the
// reference CPU path, as with the streaming kernel.
//
// Weights stream HBM -> LDS with direct-to-LDS loads in chunks of one
// superblock of a 16-row tile (16 x 144 bytes); the chunks of a workgroup's
// rows are dealt round-robin to its 8 waves, each with a D-deep ring.  The
// activation columns are staged once per workgroup in the MFMA A layout.
#include "flh_kstream.h"
#include "flh_internal.h"
#include "flh_status.h"
#include <stdio.h>
#include <stdlib.h>

namespace flh {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// Development timing probe (-DFLH_TRACE): per workgroup, s_memrealtime at
// entry, after activation staging, first chunk, last chunk and exit.
#ifdef FLH_TRACE
__device__ uint64_t g_mf_trace[8192 * 6];
#define MF_STAMP(k) do { if (threadIdx.x == 0 && blockIdx.x < 8192) \
    g_mf_trace[(size_t)blockIdx.x * 6 + (k)] = __builtin_amdgcn_s_memrealtime(); } while (0)
extern "C" int flh_mf_trace(uint64_t * host, size_t n) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_mf_trace), n * 8, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -2;
}
#else
#define MF_STAMP(k) do { } while (0)
#endif

// cache policy of the weight DMA (2 = nontemporal)
#ifndef FLH_MF_AUX
#define FLH_MF_AUX 2
#endif

constexpr uint32_t MF_WAVES = 8;
constexpr uint32_t MF_CHUNK = 2304;          // 16 rows x one Q4_K superblock
constexpr int MF_NI = 3;                     // DMA instructions per chunk

// LDS: [waves][D][2304] ring | xr [NC][XS] raw q8_K appendices | TI, TM [nl][nrb][NC]
//      | TH [nl][nrb] | ysm [nrb * NC] | (K halves) yph [nrb * NC], dkt [NC][nsb]
//      | (NC = 4, 8) zr: 128 zero bytes
// XS: a column's appendix (292 bytes per superblock) padded so that XS / 4 is
// 8 mod 32 (the 16 columns' reads of one k-slice fall in distinct banks).
//
// K halves (KH): when NC columns of nsb superblocks do not fit, the superblocks
// split by sb % 4 into half 0 ({0, 1}) and half 1 ({2, 3}); a batch streams
// one half, folds accumulators 0-1 (resp. 2-3) of the reference's four, stages
// the other half's activations and streams that.  nl = superblocks held at once.
// Term strides per superblock, padded to 8 mod 32 words: the fold's four
// accumulator lanes of a (row, column) read superblocks one apart, which would
// otherwise fall in one LDS bank (nrb * NC is a multiple of 64).
template <int NC>
__host__ __device__ inline uint32_t mf_ts(uint32_t nrb) { return nrb * NC + 8; }
__host__ __device__ inline uint32_t mf_ths(uint32_t nrb) { return nrb + 8; }
__host__ __device__ inline uint32_t mf_xs(uint32_t nsb) { return ((nsb * 292 + 127) & ~127u) + 32; }
// K halves: slot li holds its superblock's 292-byte block for each of the NC
// columns at a 304-byte pitch ([li][NC][304]), the block at byte 12 of its
// 304 (copied as 19 16-byte pieces starting 12 bytes before the block, which
// stays inside the column's q8_1 appendix for superblock 0).  A 76-word
// column pitch puts 8 columns' reads of a k-slice in distinct banks.
constexpr uint32_t MF_XB = 304, MF_XO = 12;
__host__ __device__ inline uint32_t mf_nsbh(uint32_t nsb, uint32_t h) {
    const uint32_t r = nsb & 3;
    return (nsb >> 2) * 2 + (h == 0 ? (r < 2 ? r : 2u) : (r > 2 ? r - 2 : 0u));
}
// superblock of local index li of half h
__device__ __forceinline__ uint32_t mf_sbh(uint32_t li, uint32_t h) { return 4 * (li >> 1) + 2 * h + (li & 1); }
// Activations in the chunk (XC, one 16-row tile per workgroup): each chunk's
// DMA also brings its superblock's NC activation blocks, at MF_CHUNK + [NC][304]
// of the stage (the K-halves slot layout); no whole-activation staging.  With
// one tile per workgroup every activation block is used by exactly one chunk,
// so this moves the same bytes as staging them whole, and where NC columns do
// not fit whole (8 columns x 56 superblocks are 131 KB) it replaces K halves
// (no half boundary, no restaging); the fold reads the q8_K scales from dkt.
template <int NC> __host__ __device__ constexpr uint32_t mf_xci() { return (19 * NC + 63) / 64; }
template <int NC, bool XC> __host__ __device__ constexpr uint32_t mf_stg() { return XC ? MF_CHUNK + NC * MF_XB : MF_CHUNK; }
template <int NC, bool XC> __host__ __device__ constexpr int mf_ni() { return XC ? MF_NI + (int)mf_xci<NC>() : MF_NI; }
// OWN (register accumulators, whole activations only): the parked terms are
// replaced by the per-(tile, accumulator class) sums AC[nrb / 16][4][16][NC].
template <int NC, bool KH, bool XC = false, bool OWN = false>
__host__ __device__ inline size_t mf_smem_bytes(uint32_t nrb, uint32_t nsb, int D) {
    const uint32_t nl = KH ? mf_nsbh(nsb, 0) : nsb;
    const size_t terms = OWN ? (size_t)nrb * 4 * NC * 4 : (size_t)mf_ts<NC>(nrb) * nl * 8 + (size_t)mf_ths(nrb) * nl * 4;
    return (size_t)MF_WAVES * D * mf_stg<NC, XC>() +
           (KH ? (size_t)nl * NC * MF_XB : XC ? 0 : (size_t)NC * mf_xs(nl)) + terms + (size_t)nrb * NC * 4 +
           (KH ? (size_t)nrb * NC * 4 : 0) + (KH || XC ? (size_t)NC * nsb * 4 : 0) + (NC <= 8 ? 128 : 0);
}

// Column sources of one pass: activation column p at x(p) (fp32 x followed by
// its appendices), output column p at y(p).
struct MfColsStrided {
    const float * x0;
    float * y0;
    uint32_t xs, ys;
    __device__ const float * x(uint32_t p) const { return x0 + (size_t)p * xs; }
    __device__ float * y(uint32_t p) const { return y0 + (size_t)p * ys; }
};

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Activation operands of one superblock from column r's raw q8_K block at xs:
// xw[2c + h] = bytes 36 + 64c + 32h + 8j .. +7 (sub-block 2c + h, k-slice j),
// bp = the bsum pairs of sub-blocks j and 4 + j.  Hidden from the compiler's
// wait-count pass (a plain read of DMA-written LDS would wait for every
// outstanding load); waits for its own reads.
__device__ __forceinline__ void mf_ld_x(const uint8_t * xs, uint32_t j, u32x2 (&xw)[8], u32x2 & bp) {
    const uint32_t a8 = lds_off(xs) + 8 * j, a4 = lds_off(xs) + 4 * j;
    asm volatile(
        "ds_read2_b32 %0, %9 offset0:9 offset1:10\n\t"
        "ds_read2_b32 %1, %9 offset0:17 offset1:18\n\t"
        "ds_read2_b32 %2, %9 offset0:25 offset1:26\n\t"
        "ds_read2_b32 %3, %9 offset0:33 offset1:34\n\t"
        "ds_read2_b32 %4, %9 offset0:41 offset1:42\n\t"
        "ds_read2_b32 %5, %9 offset0:49 offset1:50\n\t"
        "ds_read2_b32 %6, %9 offset0:57 offset1:58\n\t"
        "ds_read2_b32 %7, %9 offset0:65 offset1:66\n\t"
        "ds_read2_b32 %8, %10 offset0:1 offset1:5\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(xw[0]), "=&v"(xw[1]), "=&v"(xw[2]), "=&v"(xw[3]), "=&v"(xw[4]), "=&v"(xw[5]), "=&v"(xw[6]),
          "=&v"(xw[7]), "=&v"(bp)
        : "v"(a8), "v"(a4));
}

// NC = 4 (block-diagonal A): xw[4G + m] = bytes 36 + 64j + 32G + 8m .. +7 of
// the block at byte address ax - 64j (sub-block 2j + G, k-slice m); lanes off
// the diagonal pass ax = a zero region - 36.  bp = bsum pairs of sub-blocks j
// and 4 + j of the block at ab - 4j.  Waits for its own reads, as mf_ld_x.
__device__ __forceinline__ void mf_ld_x4(uint32_t ax, uint32_t ab, u32x2 (&xw)[8], u32x2 & bp) {
    asm volatile(
        "ds_read2_b32 %0, %9 offset0:9 offset1:10\n\t"
        "ds_read2_b32 %1, %9 offset0:11 offset1:12\n\t"
        "ds_read2_b32 %2, %9 offset0:13 offset1:14\n\t"
        "ds_read2_b32 %3, %9 offset0:15 offset1:16\n\t"
        "ds_read2_b32 %4, %9 offset0:17 offset1:18\n\t"
        "ds_read2_b32 %5, %9 offset0:19 offset1:20\n\t"
        "ds_read2_b32 %6, %9 offset0:21 offset1:22\n\t"
        "ds_read2_b32 %7, %9 offset0:23 offset1:24\n\t"
        "ds_read2_b32 %8, %10 offset0:1 offset1:5\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(xw[0]), "=&v"(xw[1]), "=&v"(xw[2]), "=&v"(xw[3]), "=&v"(xw[4]), "=&v"(xw[5]), "=&v"(xw[6]),
          "=&v"(xw[7]), "=&v"(bp)
        : "v"(ax), "v"(ab));
}

// NC = 8 (block-diagonal A): xw[4cc + 2n + m] = bytes 36 + 128h + 64cc + 32n +
// 16m + 8e .. +7 of the block at ax - 128h - 8e (h = j >> 1, e = j & 1: sub-block
// 4h + 2cc + n, k-slice 2m + e); lanes off the diagonal pass ax = a zero region
// - 36.  bp as mf_ld_x4.
__device__ __forceinline__ void mf_ld_x8(uint32_t ax, uint32_t ab, u32x2 (&xw)[8], u32x2 & bp) {
    asm volatile(
        "ds_read2_b32 %0, %9 offset0:9 offset1:10\n\t"
        "ds_read2_b32 %1, %9 offset0:13 offset1:14\n\t"
        "ds_read2_b32 %2, %9 offset0:17 offset1:18\n\t"
        "ds_read2_b32 %3, %9 offset0:21 offset1:22\n\t"
        "ds_read2_b32 %4, %9 offset0:25 offset1:26\n\t"
        "ds_read2_b32 %5, %9 offset0:29 offset1:30\n\t"
        "ds_read2_b32 %6, %9 offset0:33 offset1:34\n\t"
        "ds_read2_b32 %7, %9 offset0:37 offset1:38\n\t"
        "ds_read2_b32 %8, %10 offset0:1 offset1:5\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(xw[0]), "=&v"(xw[1]), "=&v"(xw[2]), "=&v"(xw[3]), "=&v"(xw[4]), "=&v"(xw[5]), "=&v"(xw[6]),
          "=&v"(xw[7]), "=&v"(bp)
        : "v"(ax), "v"(ab));
}

// up to 4 dwords at LDS addresses a[i], one wait (hidden from the compiler's
// wait-count pass, as mf_ld_x)
template <int N>
__device__ __forceinline__ void mf_ld_dk(const uint32_t (&a)[N], float (&v)[N]) {
    uint32_t r[4];
    if constexpr (N == 1) {
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(r[0]) : "v"(a[0]));
    } else if constexpr (N == 2) {
        asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1]) : "v"(a[0]), "v"(a[1]));
    } else {
        asm volatile("ds_read_b32 %0, %4\n\tds_read_b32 %1, %5\n\tds_read_b32 %2, %6\n\tds_read_b32 %3, %7\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]) : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]));
    }
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = __uint_as_float(r[i]);
}

__device__ __forceinline__ void lds_st64(void * p, u32x2 v) {
    asm volatile("ds_write_b64 %0, %1" :: "v"(lds_off(p)), "v"(v));
}

// Sum of v over the four 16-lane rows, transposed: lane row j gets
// sum over rows of p[j] (two permlane32 swaps pair rows j, j + 2; one
// permlane16 swap pairs rows j, j + 1).  Integer adds: exact in any order.
__device__ __forceinline__ int mf_rowsum_t(const int (&p)[4]) {
    const auto a = __builtin_amdgcn_permlane32_swap((uint32_t)p[0], (uint32_t)p[2], false, false);
    const auto b = __builtin_amdgcn_permlane32_swap((uint32_t)p[1], (uint32_t)p[3], false, false);
    const uint32_t u = a[0] + a[1], v = b[0] + b[1];
    const auto c = __builtin_amdgcn_permlane16_swap(u, v, false, false);
    return (int)(c[0] + c[1]);
}

// Reference-order fold of column p for the rows rl0 + FR*i, i < R (terms
// [sb][row][column]; the q8_K scale read from the column's raw appendix at
// xp): lane k runs accumulator k over superblocks k, k + 4, ...; the quad
// then combines (a0 + a1) + (a2 + a3).  Same float operations, in the same
// order, as ks_fold and fl_dot_i8k_q4_K.  The R rows' loads of four steps
// are issued together: a fold's time is its LDS round trips (~0.4 us each
// here), so R rows per round instead of one.  Rows >= nrow fold row nrow - 1
// again (their results are not stored).
template <int NC, int R>
__device__ __forceinline__ void mf_fold(const int * TI, const int * TM, const uint32_t * TH, const uint8_t * xp,
                                        uint32_t nsb, uint32_t nrb, uint32_t k, uint32_t p, uint32_t rl0, uint32_t FR,
                                        uint32_t nrow, bool fok, float (&res)[R], uint32_t xps = 292) {
    float acc[R];
    uint32_t rl[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        acc[i] = 0.f;
        rl[i] = min(rl0 + FR * i, nrow - 1);
    }
    if (fok) {
        auto step = [&](float & a, int ti, int tm, uint32_t th, float dk) {
            const float d = h2f(th & 0xFFFFu), dmin = h2f(th >> 16);
            a = fmaf(d * dk, (float)ti, a);
            a = fmaf(-(dmin * dk), (float)tm, a);
        };
        uint32_t s = k;
        for (; s + 12 < nsb; s += 16) {
            int ti[R][4], tm[R][4];
            uint32_t th[R][4];
            float dk[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t sq = s + 4 * q;
                dk[q] = *(const float *)(xp + (size_t)sq * xps);
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    ti[i][q] = TI[(size_t)sq * mf_ts<NC>(nrb) + rl[i] * NC + p];
                    tm[i][q] = TM[(size_t)sq * mf_ts<NC>(nrb) + rl[i] * NC + p];
                    th[i][q] = TH[(size_t)sq * mf_ths(nrb) + rl[i]];
                }
            }
#pragma unroll
            for (int i = 0; i < R; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) step(acc[i], ti[i][q], tm[i][q], th[i][q], dk[q]);
        }
        for (; s < nsb; s += 4) {
            const float dk = *(const float *)(xp + (size_t)s * xps);
#pragma unroll
            for (int i = 0; i < R; ++i)
                step(acc[i], TI[(size_t)s * mf_ts<NC>(nrb) + rl[i] * NC + p],
                     TM[(size_t)s * mf_ts<NC>(nrb) + rl[i] * NC + p], TH[(size_t)s * mf_ths(nrb) + rl[i]], dk);
        }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const float s01 = acc[i] + qx1f(acc[i]);
        res[i] = s01 + qx2f(s01);
    }
}

// Wait until at most n of this wave's DMA instructions are outstanding
// (n >= 15 waits for 15: more waiting, never less).
__device__ __forceinline__ void mf_wait_vm(uint32_t n) {
    // wave-uniform by construction; readfirstlane keeps the switch on the
    // scalar unit (a divergent switch runs every case's wait)
    switch (__builtin_amdgcn_readfirstlane(n)) {
        case 0: WAIT_VM(0); break;
        case 1: WAIT_VM(1); break;
        case 2: WAIT_VM(2); break;
        case 3: WAIT_VM(3); break;
        case 4: WAIT_VM(4); break;
        case 5: WAIT_VM(5); break;
        case 6: WAIT_VM(6); break;
        case 7: WAIT_VM(7); break;
        case 8: WAIT_VM(8); break;
        case 9: WAIT_VM(9); break;
        case 10: WAIT_VM(10); break;
        case 11: WAIT_VM(11); break;
        case 12: WAIT_VM(12); break;
        case 13: WAIT_VM(13); break;
        case 14: WAIT_VM(14); break;
        default: WAIT_VM(15); break;
    }
}

// K halves: fold of half h (local superblocks li, terms [li][row][column]):
// lane k < 2 runs accumulator 2h + k over li = k, k + 2, ... (superblocks in
// increasing order); returns a_{2h} + a_{2h+1} in lane 0 of the quad.  The
// q8_K scales come from dkt [column][sb].
template <int NC>
__device__ __forceinline__ float mf_fold_h(const int * TI, const int * TM, const uint32_t * TH, const float * dkt,
                                           uint32_t nl, uint32_t nsb, uint32_t h, uint32_t nrb, uint32_t k,
                                           uint32_t p, uint32_t rl, bool fok) {
    float acc = 0.f;
    if (fok && k < 2) {
        auto step = [&](int ti, int tm, uint32_t th, float dk) {
            const float d = h2f(th & 0xFFFFu), dmin = h2f(th >> 16);
            acc = fmaf(d * dk, (float)ti, acc);
            acc = fmaf(-(dmin * dk), (float)tm, acc);
        };
        uint32_t li = k;
        for (; li + 6 < nl; li += 8) {
            int ti[4], tm[4];
            uint32_t th[4];
            float dk[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t lq = li + 2 * q;
                ti[q] = TI[(size_t)lq * mf_ts<NC>(nrb) + rl * NC + p];
                tm[q] = TM[(size_t)lq * mf_ts<NC>(nrb) + rl * NC + p];
                th[q] = TH[(size_t)lq * mf_ths(nrb) + rl];
                dk[q] = dkt[p * nsb + mf_sbh(lq, h)];
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) step(ti[q], tm[q], th[q], dk[q]);
        }
        for (; li < nl; li += 2)
            step(TI[(size_t)li * mf_ts<NC>(nrb) + rl * NC + p], TM[(size_t)li * mf_ts<NC>(nrb) + rl * NC + p],
                 TH[(size_t)li * mf_ths(nrb) + rl],
                 dkt[p * nsb + mf_sbh(li, h)]);
    }
    return acc + qx1f(acc);
}

// One pass over the rows [rows*g/G, rows*(g+1)/G) for nx <= NC columns, in
// batches of nrb rows (a multiple of 16).  A chunk is superblock sb of a
// 16-row tile of the batch; the batch's chunks q = (tile, sb), tile-major, are
// dealt to the waves round-robin (with K halves: per half, the first half of
// batch bt being half bt & 1, whose activations are staged already).
template <int NC, int D, bool KH, typename COLS, bool XC = false, bool OWN = false>
__device__ __forceinline__ void mf_body(const uint8_t * __restrict__ w, uint32_t rows, uint32_t cols,
                                        const COLS & C, uint32_t nx, uint32_t nrbp, uint32_t g, uint32_t G,
                                        uint8_t * sm) {
    // nrbp: rows per batch | chunks issued before the first is consumed << 16 (0: D)
    const uint32_t nrb = nrbp & 0xFFFF;
    const uint32_t pro = (nrbp >> 16) ? min(nrbp >> 16, (uint32_t)D) : (uint32_t)D;
    const uint32_t nsb = cols >> 8;
    const uint64_t rb = (uint64_t)nsb * 144;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t r = lane & 15, j = lane >> 4;
    constexpr uint32_t NPH = KH ? 2 : 1;                          // phases (halves) per batch
    auto half_of = [&](uint32_t bt, uint32_t ph) -> uint32_t { return KH ? ((bt & 1) ^ ph) : 0u; };
    auto nl_of = [&](uint32_t h) -> uint32_t { return KH ? mf_nsbh(nsb, h) : nsb; };
    auto sb_of = [&](uint32_t li, uint32_t h) -> uint32_t { return KH ? mf_sbh(li, h) : li; };
    const uint32_t NL = nl_of(0);                                 // superblocks held at once
    static_assert(!(KH && XC), "one activation mode");
    constexpr uint32_t STG = mf_stg<NC, XC>();                   // ring stage bytes
    constexpr int NI = mf_ni<NC, XC>();                           // DMA instructions per chunk
    uint8_t * myst = sm + (size_t)wave * D * STG;
    const uint32_t XS = KH || XC ? 0u : mf_xs(NL);
    uint8_t * xr = sm + (size_t)MF_WAVES * D * STG;
    static_assert(!OWN || (!KH && !XC), "register accumulators: whole activations staged");
    int * TI = (int *)(xr + (KH ? (size_t)NL * NC * MF_XB : (size_t)NC * XS));
    int * TM = TI + (size_t)mf_ts<NC>(nrb) * NL;
    uint32_t * TH = (uint32_t *)(TM + (size_t)mf_ts<NC>(nrb) * NL);
    float * AC = (float *)TI;                                     // OWN: [nrb / 16][4][16][NC]
    float * ysm = OWN ? AC + (size_t)nrb * 4 * NC : (float *)(TH + (size_t)mf_ths(nrb) * NL);
    float * yph = ysm + (size_t)nrb * NC;                         // KH: first half's sums
    float * dkt = KH ? yph + (size_t)nrb * NC : yph;              // KH, XC: q8_K scales [NC][nsb]
    uint8_t * zr = KH || XC ? (uint8_t *)(dkt + (size_t)NC * nsb) : (uint8_t *)yph;   // NC <= 8: zeros
    // NC = 4: each MFMA's A is block-diagonal (rows 4g .. 4g + 3 = the four
    // columns on k-slice g only), so one wave's 8 MFMAs give every lane row j
    // the dots of sub-blocks 2j, 2j + 1 for the 4 columns: the scale-weighted
    // sum is 8 products plus a cross-row sum, not 32 products.  NC = 8: rows
    // 8h .. 8h + 7 on k-slices 2h, 2h + 1; lane rows 2h, 2h + 1 get sub-blocks
    // 4h .. 4h + 3 (16 products, a sum over h)
    constexpr bool BD = NC <= 8;
    if constexpr (BD) if (tid < 32) lds_st32(zr + 4 * tid, 0u);

    MF_STAMP(0);
    const uint32_t rbeg = (uint32_t)((uint64_t)rows * g / G);
    const uint32_t rend = (uint32_t)((uint64_t)rows * (g + 1) / G);
    const uint32_t nbatch = (rend - rbeg + nrb - 1) / nrb;
    auto nrow_of = [&](uint32_t bt) -> uint32_t { return min(nrb, rend - rbeg - bt * nrb); };

    // ---- activations -> LDS by DMA, issued first (older than every weight
    // DMA, so the wait before the first chunk covers them).  Whole: each
    // column's q8_K appendix copied as is, 1 KiB per instruction, the last
    // 0-12 bytes by a dword instruction.  K halves: the half's slots, 1 KiB
    // per instruction, plus every superblock's scale into dkt.  Columns past
    // nx copy column 0 (their results are never stored).
    // K halves: DMA of slots [l0, l1) of half h (19 NC pieces per slot), the
    // instructions dealt from wave w0 with stride ws; returns the number of
    // instructions this wave issued (each has an active lane).
    auto stage_slots = [&](uint32_t h, uint32_t l0, uint32_t l1, uint32_t w0, uint32_t ws) -> uint32_t {
        const uint32_t e0 = l0 * 19 * NC, e1 = l1 * 19 * NC, nin = (e1 - e0 + 63) >> 6;
        uint32_t cnt = 0;
        for (uint32_t i = w0; i < nin; i += ws) {
            const uint32_t e = e0 + 64 * i + lane;
            if (e < e1) {
                const uint32_t li = e / (19 * NC), rem = e - li * 19 * NC, n = rem / 19, o = rem - n * 19;
                const uint8_t * src = (const uint8_t *)C.x(n < nx ? n : 0) + xqk_off(cols) +
                                      (size_t)mf_sbh(li, h) * 292 + 16 * o - MF_XO;
                __builtin_amdgcn_global_load_lds(GPTR(src), LPTR(xr + 16 * (size_t)(e0 + 64 * i)), 16, 0, 0);
            }
            ++cnt;
        }
        return cnt;
    };
    if constexpr (KH || XC) {
        if constexpr (KH) stage_slots(0, 0, nl_of(0), wave, MF_WAVES);
        for (uint32_t i = wave; i < (NC * nsb + 63) / 64; i += MF_WAVES) {
            const uint32_t e = 64 * i + lane;
            if (e < NC * nsb) {
                const uint32_t n = e / nsb, sb = e - n * nsb;
                const uint8_t * src = (const uint8_t *)C.x(n < nx ? n : 0) + xqk_off(cols) + (size_t)sb * 292;
                __builtin_amdgcn_global_load_lds(GPTR(src), LPTR(dkt + 64 * i), 4, 0, 0);
            }
        }
    } else {
        const uint32_t L = nsb * 292, n16 = L >> 4, nti = (n16 + 63) >> 6;   // x4 instructions per column
        const uint32_t tail = (L & 15) >> 2;                                  // trailing dwords
        const uint32_t per = nti + (tail ? 1u : 0u);
        for (uint32_t i = wave; i < NC * per; i += MF_WAVES) {
            const uint32_t n = i / per, k = i % per;
            const uint8_t * src = (const uint8_t *)C.x(n < nx ? n : 0) + xqk_off(cols);
            uint8_t * dst = xr + (size_t)n * XS;
            if (k < nti) {
                const uint32_t pc = 64 * k + lane;
                if (pc < n16) __builtin_amdgcn_global_load_lds(GPTR(src + 16 * pc), LPTR(dst + 1024 * k), 16, 0, 0);
            } else if (lane < tail) {
                __builtin_amdgcn_global_load_lds(GPTR(src + 16 * n16 + 4 * lane), LPTR(dst + 16 * n16), 4, 0, 0);
            }
        }
    }

    // ---- weight chunk stream.  Per-lane DMA pieces: piece p (16 bytes) of a
    // chunk is row p / 9, bytes 16 (p % 9) of its superblock.
    const uint32_t pr0 = lane / 9, pr1 = (64 + lane) / 9, pr2 = (128 + (lane >> 2)) / 9;
    const uint32_t po0 = (lane % 9) * 16, po1 = ((64 + lane) % 9) * 16, po2 = ((128 + (lane >> 2)) % 9) * 16 + 4 * (lane & 3);
    // issue cursor: batch qbt, phase qph, tile qt, local superblock qsb
    // (q = wave + 8 i over the phase's chunks, tile-major)
    // OWN: wave w owns accumulator class k = w % 4 (superblocks k, k + 4, ...
    // of a tile, in order) of the tiles t = w / 4, w / 4 + 2, ...; otherwise
    // the phase's chunks q = wave + 8 i, tile-major
    const uint32_t own_k = wave & 3, own_t = wave >> 2;
    auto cur_first = [&](uint32_t & t, uint32_t & sb, uint32_t nl) {
        if constexpr (OWN) {
            t = own_t;
            sb = own_k;
        } else {
            t = 0;
            sb = wave;
            while (sb >= nl) { sb -= nl; ++t; }
        }
    };
    auto cur_next = [&](uint32_t & t, uint32_t & sb, uint32_t nl) {
        if constexpr (OWN) {
            sb += 4;
            if (sb >= nl) { sb = own_k; t += 2; }
        } else {
            sb += MF_WAVES;
            while (sb >= nl) { sb -= nl; ++t; }
        }
    };
    uint32_t qbt = 0, qph = 0, qt = 0, qsb = 0, qnl = nl_of(half_of(0, 0));
    uint32_t qnt = nbatch ? (nrow_of(0) + 15) >> 4 : 0;
    cur_first(qt, qsb, qnl);
    uint32_t nissued = 0, ncons = 0;
    // K halves: this wave's DMA instructions so far (vm), and that count right
    // after each ring stage's chunk, the y DMA and the latest restaging: the
    // restaging DMAs interleave with the chunks, so waits count instructions
    uint32_t vm = 0, ce0 = 0, ce1 = 0, y_vm = 0, rs_vm = 0;
    // one slot's restaging: per instruction i, this lane's piece (column, 16-byte
    // offset) is fixed, so its source minus the superblock offset is kept
    constexpr uint32_t NIR = (19 * NC + 63) / 64;                 // instructions per slot
    const uint8_t * rsrc[NIR];
#pragma unroll
    for (uint32_t i = 0; i < NIR; ++i) {
        const uint32_t pc = 64 * i + lane, n = pc / 19, o = pc - n * 19;
        rsrc[i] = (const uint8_t *)C.x(n < nx && n < NC ? n : 0) + xqk_off(cols) + 16 * o - MF_XO;
    }
    auto restage_slot = [&](uint32_t h, uint32_t li) {
        const size_t so = (size_t)mf_sbh(li, h) * 292;
#pragma unroll
        for (uint32_t i = 0; i < NIR; ++i)
            if (64 * i + lane < 19 * NC)
                __builtin_amdgcn_global_load_lds(GPTR(rsrc[i] + so), LPTR(xr + 16 * (size_t)li * 19 * NC + 1024 * i),
                                                 16, 0, 0);
        vm += NIR;
    };
    static_assert(!KH || D == 2, "K halves run a 2-deep ring");
    auto issue_one = [&]() {
        while (qbt < nbatch && qt >= qnt) {
            if (++qph == NPH) {
                qph = 0;
                ++qbt;
                qnt = qbt < nbatch ? (nrow_of(qbt) + 15) >> 4 : 0;
            }
            qnl = nl_of(half_of(qbt, qph));
            cur_first(qt, qsb, qnl);
        }
        if (qbt < nbatch) {
            const uint32_t tr0 = rbeg + qbt * nrb + 16 * qt;
            const uint32_t nv1 = min(16u, rend - tr0) - 1;           // last valid row of the tile
            const uint8_t * base = w + (size_t)tr0 * rb + (size_t)sb_of(qsb, half_of(qbt, qph)) * 144;
            uint8_t * stage = myst + (nissued % D) * STG;
            __builtin_amdgcn_global_load_lds(GPTR(base + (size_t)min(pr0, nv1) * rb + po0), LPTR(stage), 16, 0, FLH_MF_AUX);
            __builtin_amdgcn_global_load_lds(GPTR(base + (size_t)min(pr1, nv1) * rb + po1), LPTR(stage + 1024), 16, 0,
                                             FLH_MF_AUX);
            __builtin_amdgcn_global_load_lds(GPTR(base + (size_t)min(pr2, nv1) * rb + po2), LPTR(stage + 2048), 4, 0,
                                             FLH_MF_AUX);
            if constexpr (XC) {
                const size_t so = (size_t)sb_of(qsb, half_of(qbt, qph)) * 292;
#pragma unroll
                for (uint32_t i = 0; i < NIR; ++i)
                    if (64 * i + lane < 19 * NC)
                        __builtin_amdgcn_global_load_lds(GPTR(rsrc[i] + so), LPTR(stage + MF_CHUNK + 1024 * i), 16, 0,
                                                         0);
            }
            if constexpr (KH) {
                vm += MF_NI;
                ce1 = (nissued & 1) ? vm : ce1;
                ce0 = (nissued & 1) ? ce0 : vm;
            }
            ++nissued;
            cur_next(qt, qsb, qnl);
        }
    };
    // old y of a batch -> LDS (one 64-float DMA per wave; nrb * NC <= 512)
    bool y_mine = false;
    uint32_t y_at = 0;
    auto issue_y = [&](uint32_t bt) {
        const uint32_t row0 = rbeg + bt * nrb, nrow = nrow_of(bt);
        y_mine = wave * 64 < nrow * NC;
        if (y_mine) {
            const uint32_t e = wave * 64 + lane, yr = e / NC, yp = e % NC;
            const bool yv = yr < nrow && yp < nx;
            const float * ya = yv ? C.y(yp) + row0 + yr : C.y(0) + row0;
            __builtin_amdgcn_global_load_lds(GPTR(ya), LPTR(ysm + wave * 64), 4, 0, 0);
            y_at = nissued;
            y_vm = ++vm;
        }
    };
    if (nbatch) issue_y(0);
    // the first pro chunks now (a smaller launch-time burst), the rest of the
    // ring after the first chunk is consumed
    for (uint32_t k = 0; k < pro; ++k) issue_one();
    // the activation and y DMAs are older than the nissued chunks
    ks_wait_behind<NI, D + 1>(nissued);
    lds_barrier();
    MF_STAMP(1);

    const uint32_t fk = tid & 3, fp = (tid >> 2) % NC, frl0 = tid / (4 * NC);
    // OWN: this lane's running sums of accumulator class own_k for its NCL
    // (row r, column c0 + i) pairs of the current tile, in the reference's
    // fmaf order (fl_dot_i8k_q4_K, src/runtime/quants.h:538-561), stored to
    // AC after the class's last superblock of the tile
    constexpr int NCL = NC == 4 ? 1 : NC == 8 ? 2 : 4;
    float acc_o[NCL];
#pragma unroll
    for (int i = 0; i < NCL; ++i) acc_o[i] = 0.f;
    auto own_step = [&](const int (&ti)[NCL], const float (&tm)[NCL], uint32_t c0, uint32_t hdx, uint32_t li,
                        uint32_t nl, uint32_t t) {
        const float d = h2f(hdx & 0xFFFFu), dmin = h2f(hdx >> 16);
        uint32_t da[NCL];
#pragma unroll
        for (int i = 0; i < NCL; ++i) da[i] = lds_off(xr + (size_t)(c0 + i) * XS + (size_t)li * 292);
        float dk[NCL];
        mf_ld_dk<NCL>(da, dk);
        if (li == own_k) {
#pragma unroll
            for (int i = 0; i < NCL; ++i) acc_o[i] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < NCL; ++i) {
            acc_o[i] = fmaf(d * dk[i], (float)ti[i], acc_o[i]);
            acc_o[i] = fmaf(-(dmin * dk[i]), tm[i], acc_o[i]);
        }
        if (li + 4 >= nl) {
            float * ap = AC + ((size_t)(t * 4 + own_k) * 16 + r) * NC + c0;
            if constexpr (NCL == 1) lds_st32(ap, __float_as_uint(acc_o[0]));
            else if constexpr (NCL == 2) lds_st64(ap, u32x2{__float_as_uint(acc_o[0]), __float_as_uint(acc_o[1])});
            else lds_st128(ap, u32x4a{__float_as_uint(acc_o[0]), __float_as_uint(acc_o[1]),
                                      __float_as_uint(acc_o[2]), __float_as_uint(acc_o[3])});
        }
    };
    constexpr uint32_t FROWS = MF_WAVES * 64 / (4 * NC);         // rows folded per pass
    uint32_t slot = 0;
    for (uint32_t bt = 0; bt < nbatch; ++bt) {
        const uint32_t row0 = rbeg + bt * nrb;
        const uint32_t nrow = nrow_of(bt);
        const uint32_t nt = (nrow + 15) >> 4;
        if (bt != 0) issue_y(bt);
        for (uint32_t ph = 0; ph < NPH; ++ph) {
            const uint32_t h = half_of(bt, ph), nl = nl_of(h);
            uint32_t ct = 0, csb = 0;                              // consume cursor
            cur_first(ct, csb, nl);
            // K halves: a slot is restaged right after its last use when one
            // wave consumes every chunk of that slot (one tile, or nl a
            // multiple of the wave count); otherwise after the half
            const bool early = nt == 1 || nl % MF_WAVES == 0;
            if constexpr (KH) {
                // slots of the other half that this half does not use are
                // free now: stage them (waves by slot)
                const uint32_t nlo = nl_of(h ^ 1);
                for (uint32_t li = nl + wave; early && ph == 0 && li < nlo; li += MF_WAVES) {
                    restage_slot(h ^ 1, li);
                    rs_vm = vm;
                }
            }
            for (; ct < nt;) {
                if constexpr (KH) mf_wait_vm(vm - (((ncons & 1) ? ce1 : 0u) | ((ncons & 1) ? 0u : ce0)));
                else ks_wait_behind<NI, D>(nissued - 1 - ncons);
                ++ncons;
                if (ncons == 1) MF_STAMP(2);
                const uint32_t t = ct, li = csb;
                cur_next(ct, csb, nl);
                const uint8_t * rp = myst + slot * STG + 144 * r;
                const uint8_t * xs_c = myst + slot * STG + MF_CHUNK + MF_XO;   // XC: column blocks, 304 B apart
                const u32x4a hd = *(const u32x4a *)rp;
                uint32_t qw[4][2];
                u32x4a qv[2];                                       // NC = 4: qs bytes 32j .. 32j + 31
                u32x2 qb[4];                                        // NC = 8: qs bytes 64h + 32cc + 16m + 8e
                if constexpr (NC == 4) {
                    qv[0] = *(const u32x4a *)(rp + 16 + 32 * j);
                    qv[1] = *(const u32x4a *)(rp + 32 + 32 * j);
                } else if constexpr (NC == 8) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) qb[q] = *(const u32x2 *)(rp + 16 + 64 * (j >> 1) + 16 * q + 8 * (j & 1));
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        qw[c][0] = *(const uint32_t *)(rp + 16 + 32 * c + 8 * j);
                        qw[c][1] = *(const uint32_t *)(rp + 20 + 32 * c + 8 * j);
                    }
                }
                // activation operands of this superblock (zero for lanes past NC):
                // column r, bytes 32g + 8j .. +7 of sub-block g; sub-block sums
                // bsum[2g] + bsum[2g + 1] for g = j and 4 + j
                u32x2 xw[8] = {};
                u32x2 bp = {};
                if constexpr (BD) {
                    // column r % NC (rows NC .. 15 of the min term are never stored)
                    const uint32_t ab = lds_off(XC ? xs_c + (size_t)(r & (NC - 1)) * MF_XB
                                                : KH ? xr + ((size_t)li * NC + (r & (NC - 1))) * MF_XB + MF_XO
                                                     : xr + (size_t)(r & (NC - 1)) * XS + (size_t)li * 292);
                    if constexpr (NC == 4)
                        mf_ld_x4((r >> 2) == j ? ab + 64 * j : lds_off(zr) - 36, ab + 4 * j, xw, bp);
                    else
                        mf_ld_x8((r >> 3) == (j >> 1) ? ab + 128 * (j >> 1) + 8 * (j & 1) : lds_off(zr) - 36, ab + 4 * j,
                                 xw, bp);
                } else if (r < NC)
                    mf_ld_x(XC ? xs_c + (size_t)r * MF_XB
                               : KH ? xr + ((size_t)li * NC + r) * MF_XB + MF_XO : xr + (size_t)r * XS + (size_t)li * 292,
                            j, xw, bp);
                const uint32_t bp0 = bp.x, bp1 = bp.y;
                // every read of this stage is done before it is refilled
                WAIT_LGKM0();
                if constexpr (KH) {
                    // the slot's last use in this half: stage the other half's
                    // block into it (ahead of the next chunk, so chunk waits
                    // count it)
                    if (early && ph == 0 && t == nt - 1 && li < nl_of(h ^ 1)) {
                        restage_slot(h ^ 1, li);
                        rs_vm = vm;
                    }
                }
                issue_one();
                if (ncons == 1)
                    for (uint32_t k = 1; k < (uint32_t)D; ++k)
                        if (nissued < ncons + D) issue_one();
                slot = slot + 1 == (uint32_t)D ? 0 : slot + 1;

                // scales / mins of row r (6-bit, SWAR as in fl_q4k_scale_min)
                const uint32_t sclo = hd.y & 0x3F3F3F3Fu, mlo = hd.z & 0x3F3F3F3Fu;
                const uint32_t schi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
                const uint32_t mhi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
                v4i acc[8];
                v4i a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};           // NC = 4: sub-blocks 2j, 2j + 1
                v4i ab8[4] = {};                                    // NC = 8: sub-blocks 4h + sl
                if constexpr (NC == 8) {
#pragma unroll
                    for (int q = 0; q < 8; ++q) {                   // q = 4cc + 2n + m
                        const u32x2 b = qb[2 * (q >> 2) + (q & 1)];
                        const uint32_t b0 = (q & 2) ? (b.x >> 4) & 0x0F0F0F0Fu : b.x & 0x0F0F0F0Fu;
                        const uint32_t b1 = (q & 2) ? (b.y >> 4) & 0x0F0F0F0Fu : b.y & 0x0F0F0F0Fu;
                        ab8[q >> 1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                            __builtin_bit_cast(long, xw[q]), (long)(((uint64_t)b1 << 32) | b0), ab8[q >> 1], 0, 0, 0);
                    }
                } else if constexpr (NC == 4) {
                    const uint32_t q[8] = {qv[0].x, qv[0].y, qv[0].z, qv[0].w, qv[1].x, qv[1].y, qv[1].z, qv[1].w};
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        const uint32_t lo0 = q[2 * m] & 0x0F0F0F0Fu, lo1 = q[2 * m + 1] & 0x0F0F0F0Fu;
                        const uint32_t hi0 = (q[2 * m] >> 4) & 0x0F0F0F0Fu, hi1 = (q[2 * m + 1] >> 4) & 0x0F0F0F0Fu;
                        a0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, xw[m]),
                                                                    (long)(((uint64_t)lo1 << 32) | lo0), a0, 0, 0, 0);
                        a1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, xw[4 + m]),
                                                                    (long)(((uint64_t)hi1 << 32) | hi0), a1, 0, 0, 0);
                    }
                } else
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const uint32_t lo0 = qw[c][0] & 0x0F0F0F0Fu, lo1 = qw[c][1] & 0x0F0F0F0Fu;
                    const uint32_t hi0 = (qw[c][0] >> 4) & 0x0F0F0F0Fu, hi1 = (qw[c][1] >> 4) & 0x0F0F0F0Fu;
                    const long blo = (long)(((uint64_t)lo1 << 32) | lo0), bhi = (long)(((uint64_t)hi1 << 32) | hi0);
                    const long alo = __builtin_bit_cast(long, xw[2 * c]);
                    const long ahi = __builtin_bit_cast(long, xw[2 * c + 1]);
                    acc[2 * c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(alo, blo, v4i{0, 0, 0, 0}, 0, 0, 0);
                    acc[2 * c + 1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ahi, bhi, v4i{0, 0, 0, 0}, 0, 0, 0);
                }
                // min term: A = sub-block sums of column r (g = 4h + j), B = mins of row r
                const float bsa0 = (float)((int)(int16_t)(bp0 & 0xFFFFu) + (int)(int16_t)(bp0 >> 16));
                const float bsa1 = (float)((int)(int16_t)(bp1 & 0xFFFFu) + (int)(int16_t)(bp1 >> 16));
                const float bm0 = (float)((mlo >> (8 * j)) & 0xFFu), bm1 = (float)((mhi >> (8 * j)) & 0xFFu);
                v4f cm = __builtin_amdgcn_mfma_f32_16x16x4f32(bsa0, bm0, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                cm = __builtin_amdgcn_mfma_f32_16x16x4f32(bsa1, bm1, cm, 0, 0, 0);
                // park: terms [li][row][column]
                const uint32_t rl = 16 * t + r;                     // row within the batch
                if constexpr (NC == 8) {
                    const uint32_t wsc = j < 2 ? sclo : schi;
                    const int s0 = (int)(wsc & 0xFFu), s1 = (int)((wsc >> 8) & 0xFFu);
                    const int s2 = (int)((wsc >> 16) & 0xFFu), s3 = (int)(wsc >> 24);
                    int pr[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        pr[i] = __mul24(s0, ab8[0][i]) + __mul24(s1, ab8[1][i]) + __mul24(s2, ab8[2][i]) +
                                __mul24(s3, ab8[3][i]);
                    // lane rows 2h + e hold columns 4e + i of half h; the sum over h
                    // leaves columns 4e + 2h, 4e + 2h + 1 in lane row 2h + e
                    const auto u = __builtin_amdgcn_permlane32_swap((uint32_t)pr[0], (uint32_t)pr[2], false, false);
                    const auto v = __builtin_amdgcn_permlane32_swap((uint32_t)pr[1], (uint32_t)pr[3], false, false);
                    if constexpr (OWN) {
                        // min terms: lane row j holds columns 4 (j & 1) + i
                        const int ti[NCL] = {(int)(u[0] + u[1]), (int)(v[0] + v[1])};
                        const float tm[NCL] = {(j >> 1) ? cm[2] : cm[0], (j >> 1) ? cm[3] : cm[1]};
                        own_step(ti, tm, 4 * (j & 1) + 2 * (j >> 1), hd.x, li, nl, t);
                        continue;
                    }
                    const size_t e = (size_t)li * mf_ts<NC>(nrb) + rl * NC;
                    lds_st64(&TI[e + 4 * (j & 1) + 2 * (j >> 1)], u32x2{u[0] + u[1], v[0] + v[1]});
                    if (j < 2)
                        lds_st128(&TM[e + 4 * j], u32x4a{(uint32_t)(int)cm[0], (uint32_t)(int)cm[1],
                                                          (uint32_t)(int)cm[2], (uint32_t)(int)cm[3]});
                    if (j == 0) lds_st32(&TH[(size_t)li * mf_ths(nrb) + rl], hd.x);
                    continue;
                }
                if constexpr (NC == 4) {
                    const uint32_t wsc = j < 2 ? sclo : schi, sh = 16 * (j & 1);
                    const int s0 = (int)((wsc >> sh) & 0xFFu), s1 = (int)((wsc >> (sh + 8)) & 0xFFu);
                    int pr[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) pr[i] = __mul24(s0, a0[i]) + __mul24(s1, a1[i]);
                    if constexpr (OWN) {
                        // every lane row holds the min terms of columns 0..3
                        const int ti[NCL] = {mf_rowsum_t(pr)};
                        const float tm[NCL] = {j == 0 ? cm[0] : j == 1 ? cm[1] : j == 2 ? cm[2] : cm[3]};
                        own_step(ti, tm, j, hd.x, li, nl, t);
                        continue;
                    }
                    const size_t e = (size_t)li * mf_ts<NC>(nrb) + rl * NC;
                    lds_st32(&TI[e + j], (uint32_t)mf_rowsum_t(pr));
                    if (j == 0)
                        lds_st128(&TM[e], u32x4a{(uint32_t)(int)cm[0], (uint32_t)(int)cm[1], (uint32_t)(int)cm[2],
                                                  (uint32_t)(int)cm[3]});
                    if (j == 0) lds_st32(&TH[(size_t)li * mf_ths(nrb) + rl], hd.x);
                    continue;
                }
                int sc[8];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    sc[k] = (int)((sclo >> (8 * k)) & 0xFFu);
                    sc[4 + k] = (int)((schi >> (8 * k)) & 0xFFu);
                }
                // the lane's 4 columns in one 16-byte store (rows past the
                // batch and columns past nx hold values the fold never reads)
                int ia[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    ia[i] = 0;
#pragma unroll
                    for (int k = 0; k < 8; ++k) ia[i] += __mul24(sc[k], acc[k][i]);
                }
                if constexpr (OWN) {
                    if constexpr (NC == 16) {
                        const int ti[NCL] = {ia[0], ia[1], ia[2], ia[3]};
                        const float tm[NCL] = {cm[0], cm[1], cm[2], cm[3]};
                        own_step(ti, tm, 4 * j, hd.x, li, nl, t);
                    }
                    continue;
                }
                if (4 * j < NC) {
                    const size_t e = (size_t)li * mf_ts<NC>(nrb) + rl * NC + 4 * j;
                    lds_st128(&TI[e], u32x4a{(uint32_t)ia[0], (uint32_t)ia[1], (uint32_t)ia[2], (uint32_t)ia[3]});
                    lds_st128(&TM[e], u32x4a{(uint32_t)(int)cm[0], (uint32_t)(int)cm[1], (uint32_t)(int)cm[2],
                                              (uint32_t)(int)cm[3]});
                }
                if (j == 0) lds_st32(&TH[(size_t)li * mf_ths(nrb) + rl], hd.x);
            }
            if constexpr (KH) {
                if (ph == 0) {
                    // this half's terms are complete and its activations read
                    lds_barrier();
                    if (!early)
                        for (uint32_t li = wave; li < nl_of(h ^ 1); li += MF_WAVES) {
                            restage_slot(h ^ 1, li);
                            rs_vm = vm;
                        }
                    for (uint32_t frl = frl0; frl < nrow; frl += FROWS) {
                        const float s0 = mf_fold_h<NC>(TI, TM, TH, dkt, nl, nsb, h, nrb, fk, fp, frl, fp < nx);
                        if (fk == 0) lds_st32(&yph[frl * NC + fp], __float_as_uint(s0));
                    }
                    // this wave's restaging has landed (the fold ran while it
                    // was in flight); the barrier publishes every wave's and
                    // orders the fold before the next half's parks
                    mf_wait_vm(vm - rs_vm);
                    lds_barrier();
                }
            }
        }
        if (!KH && y_mine) ks_wait_behind<NI, D + 1>(min(nissued - y_at, (uint32_t)D));
        if (KH && y_mine) mf_wait_vm(vm - y_vm);
        lds_barrier();
        MF_STAMP(3);
        for (uint32_t frl = frl0; KH && frl < nrow; frl += FROWS) {
            const bool fok = fp < nx;
            if constexpr (KH) {
                // (a0 + a1) + (a2 + a3): the two halves' sums in either order
                const uint32_t h1 = half_of(bt, 1);
                const float s1 = mf_fold_h<NC>(TI, TM, TH, dkt, nl_of(h1), nsb, h1, nrb, fk, fp, frl, fok);
                if (fok && fk == 0) C.y(fp)[row0 + frl] = ysm[frl * NC + fp] + (yph[frl * NC + fp] + s1);
            }
        }
        if constexpr (OWN) {
            // (a0 + a1) + (a2 + a3) of every (row, column), one per thread
            const uint32_t frl = tid / NC, p = tid % NC;
            if (frl < nrow && p < nx) {
                const float * ap = AC + ((size_t)((frl >> 4) * 4) * 16 + (frl & 15)) * NC + p;
                uint32_t aa[4] = {lds_off(ap), lds_off(ap + 16 * NC), lds_off(ap + 32 * NC), lds_off(ap + 48 * NC)};
                float av[4];
                mf_ld_dk<4>(aa, av);
                C.y(p)[row0 + frl] = ysm[frl * NC + p] + ((av[0] + av[1]) + (av[2] + av[3]));
            }
        } else if constexpr (!KH) {
            // every row of the batch in one call (nrow <= nrb <= 512 / NC = 4 FROWS)
            const bool fok = fp < nx;
            const uint8_t * xp = XC ? (const uint8_t *)(dkt + (size_t)fp * nsb) : xr + (size_t)fp * XS;
            auto fold_store = [&](auto & rr) {
                constexpr int R = sizeof(rr) / sizeof(float);
                mf_fold<NC, R>(TI, TM, TH, xp, nsb, nrb, fk, fp, frl0, FROWS, nrow, fok, rr, XC ? 4u : 292u);
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    const uint32_t frl = frl0 + FROWS * i;
                    if (fok && fk == 0 && frl < nrow) C.y(fp)[row0 + frl] = ysm[frl * NC + fp] + rr[i];
                }
            };
            if (nrow <= FROWS) {
                float rr[1];
                fold_store(rr);
            } else if (nrow <= 2 * FROWS) {
                float rr[2];
                fold_store(rr);
            } else {
                float rr[4];
                fold_store(rr);
            }
        }
        lds_barrier();
    }
    WAIT_VM(0);
    MF_STAMP(4);
}

template <int NC, int D, bool KH, bool XC = false, bool OWN = false>
__global__ __launch_bounds__(512) void k_dot_mfma(DotArgs a, uint32_t nrb) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
    const uint8_t * w = a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0);
    const MfColsStrided C{a.x, a.y, a.xstride, a.ystride};
    mf_body<NC, D, KH, MfColsStrided, XC, OWN>(w, a.rows, a.cols, C, a.nx, nrb, blockIdx.x, gridDim.x, sm);
}

// Grouped expert matvec (MoE): the routed experts share the grid (moe_assign).  The workgroup collects
// the (token, slot) pairs routed to e and streams e's weights once per group
// of NC pairs (the columns); with no pair routed to e it exits before any
// weight byte is requested.  Column p's activation index and output index
// sit in LDS tables read with the lane's own (lane-varying) p.
struct MfColsMoe {
    const float * x0;
    float * y0;
    uint32_t xs, ys;
    const uint32_t * xi;                      // __shared__ [NC]
    const uint32_t * yi;                      // __shared__ [NC]
    __device__ const float * x(uint32_t p) const { return x0 + (size_t)lds_ld32(&xi[p]) * xs; }
    __device__ float * y(uint32_t p) const { return y0 + (size_t)lds_ld32(&yi[p]) * ys; }
};

template <int NC, int D, bool KH, bool OWN = false>
__global__ __launch_bounds__(512) void k_moe_mfma(MoeArgs a, uint32_t nrbp) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
    __shared__ uint32_t pairs[256];
    __shared__ uint32_t npairs;
    __shared__ uint32_t cxi[NC], cyi[NC];
    const uint32_t tid = threadIdx.x;
    __shared__ uint32_t rids[256];
    if (tid == 0) npairs = 0;
    const uint32_t * ids = moe_route(a, rids);
    uint32_t g, G;
    const uint32_t e = moe_assign(ids, a.ntok * a.top_k, a.n_expert, blockIdx.y * gridDim.x + blockIdx.x,
                                  gridDim.x * gridDim.y, g, G);                 // (barriers)
    if (e >= a.n_expert) return;
    // pairs i = tok * top_k + slot routed to e (order free: every column's
    // output is computed independently)
    if (tid < a.ntok * a.top_k && ids[tid] == e) pairs[atomicAdd(&npairs, 1u)] = tid;
    __syncthreads();
    const uint32_t np = npairs;
    const uint8_t * w = a.w + (size_t)e * a.estride;
    for (uint32_t p0 = 0; p0 < np; p0 += NC) {
        const uint32_t nx = min((uint32_t)NC, np - p0);
        if (tid < NC) {
            const uint32_t ts = pairs[p0 + (tid < nx ? tid : 0)];
            cxi[tid] = a.x_per_slot ? ts : ts / a.top_k;
            cyi[tid] = ts;
        }
        __syncthreads();
        const MfColsMoe C{a.x, a.y, a.xstride, a.ystride, cxi, cyi};
        mf_body<NC, D, KH, MfColsMoe, false, OWN>(w, a.rows, a.cols, C, nx, nrbp, g, G, sm);
        __syncthreads();
    }
}

// ----------------------------------------------------------------- launch --
// chunks each wave requests before the activations are staged (the rest of
// its ring after its first chunk); 0 = the whole ring (measured best here)
static uint32_t mf_pro() { return tune().mf_pro; }          // 0: the whole ring
// Register accumulators (a wave owns one accumulator class of its tiles, no
// parked terms, no fold pass) where the whole activations are staged, a class
// has a superblock (nsb >= 4) and a batch holds at least two 16-row tiles
// (with one, the waves of the second tile parity would idle: verify N = 4 at
// 4096x14336, 16 rows per workgroup, 10.95 -> 12.15 us); measured at
// 14336x4096: N = 4 10.94 -> 10.24 us, N = 8 12.82 -> 11.33 us.
// FLH_MFMA_OWN=0: the parked-term fold everywhere.
static bool mf_own(uint32_t nsb, uint32_t nrb) { return tune().mf_own && nsb >= 4 && nrb >= 32; }
template <int NC, int D, bool KH, bool XC = false, bool OWN = false>
static int mf_launch_d(const DotArgs & a, uint32_t nrb, uint32_t grid, size_t smb, hipStream_t s) {
    if (int rc = lds_fits((const void *)k_dot_mfma<NC, D, KH, XC, OWN>, smb, "k_dot_mfma: LDS over the limit")) return rc;
    (void)hipFuncSetAttribute((const void *)k_dot_mfma<NC, D, KH, XC, OWN>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)smb);
    hipLaunchKernelGGL((k_dot_mfma<NC, D, KH, XC, OWN>), dim3(grid), dim3(MF_WAVES * 64), smb, s, a,
                       nrb | (mf_pro() << 16));
    return hip_check(hipGetLastError(), "k_dot_mfma launch");
}

size_t lds_limit();


// LDS plan for NC columns: one workgroup per CU, batch of nrb rows (a multiple
// of 16), ring depth D, whole activations or K halves (kh) when the whole
// activations do not fit with a 16-row batch; FLH_ERR_UNSUPPORTED if neither
// fits.
template <int NC>
static int mf_plan_kh(uint32_t rows, uint32_t nsb, uint32_t G, uint32_t & nrb, int & D, bool & kh, size_t & smb,
                      bool allow_kh = true, bool * xc = nullptr, bool * own = nullptr) {
    const size_t lim = lds_limit() - 4096;                    // the MoE kernel's static tables
    const uint32_t rpw = (rows + G - 1) / G;
    // a batch's old y values are one 64-float DMA per wave: nrb * NC <= 512
    nrb = ((rpw + 15) / 16) * 16;
    if (nrb > 512 / NC) nrb = 512 / NC;
    // measured: a 2-deep ring with a full prologue beats deeper rings (N=4,
    // 14336x4096: D=2 11.7 us, D=3 12.4 us, D=4 13.0 us)
    D = 2;
    const Tune & t = tune();
    if (t.mf_D >= 2 && t.mf_D <= 3) D = (int)t.mf_D;          // development sweeps
    if (t.mf_nrb >= 16 && t.mf_nrb % 16 == 0 && t.mf_nrb <= 512 / NC) nrb = t.mf_nrb;
    const int force_kh = t.mf_kh;
    kh = force_kh == 1 || (force_kh != 0 && mf_smem_bytes<NC, false>(16, nsb, 2) > lim);
    // K halves need at least 8 superblocks per row, and the grouped (MoE)
    // planner allows them only as a last resort
    if (kh && (nsb < 8 || (!allow_kh && force_kh != 1))) kh = false;
    // one 16-row tile per workgroup where K halves would be needed: the
    // activations ride in the chunks instead (Tune::mf_xc = false: off)
    if (xc) *xc = false;
    if (xc && kh && force_kh != 1 && t.mf_xc && nrb == 16) {
        if (mf_smem_bytes<NC, false, true>(16, nsb, 2) <= lim) {
            *xc = true;
            kh = false;
            D = 2;
            smb = mf_smem_bytes<NC, false, true>(16, nsb, 2);
            return FLH_OK;
        }
    }
    if (kh) D = 2;                                            // the K-halves waits assume it
    // register accumulators: no parked terms, so the batch can stay large
    if (own) *own = false;
    if (own && !kh && D == 2) {
        uint32_t n = nrb;
        while (mf_smem_bytes<NC, false, false, true>(n, nsb, 2) > lim && n > 16) n -= 16;
        if (mf_own(nsb, n) && mf_smem_bytes<NC, false, false, true>(n, nsb, 2) <= lim) {
            nrb = n;
            *own = true;
            smb = mf_smem_bytes<NC, false, false, true>(n, nsb, 2);
            return FLH_OK;
        }
    }
    auto bytes = [&]() { return kh ? mf_smem_bytes<NC, true>(nrb, nsb, D) : mf_smem_bytes<NC, false>(nrb, nsb, D); };
    while (bytes() > lim && nrb > 16) nrb -= 16;
    while (bytes() > lim && D > 2) --D;
    smb = bytes();
    return smb > lim ? FLH_ERR_UNSUPPORTED : FLH_OK;
}

// The plan mf_launch<NC> takes for rows x cols with nx columns (NC as in
// launch_dot_mfma): out = {K halves, activations in the chunk, nrb, D}.
int mfma_plan(uint32_t rows, uint32_t cols, uint32_t nx, uint32_t * out) {
    const uint32_t nsb = cols >> 8;
    if (nsb == 0 || (cols & 255) || nsb > 64 || nx < 1 || nx > 16 || rows == 0) return FLH_ERR_UNSUPPORTED;
    const uint32_t G = rows < (uint32_t)num_cus() ? rows : (uint32_t)num_cus();
    uint32_t nrb;
    int D;
    bool kh, xc;
    size_t smb;
    const int rc = nx <= 4 ? mf_plan_kh<4>(rows, nsb, G, nrb, D, kh, smb, true, &xc)
                 : nx <= 8 ? mf_plan_kh<8>(rows, nsb, G, nrb, D, kh, smb, true, &xc)
                           : mf_plan_kh<16>(rows, nsb, G, nrb, D, kh, smb, true, &xc);
    if (rc) return FLH_ERR_UNSUPPORTED;
    out[0] = kh;
    out[1] = xc;
    out[2] = nrb;
    out[3] = (uint32_t)D;
    return FLH_OK;
}

template <int NC>
static int mf_launch(const DotArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    const uint32_t G = a.rows < (uint32_t)num_cus() ? a.rows : (uint32_t)num_cus();
    uint32_t nrb;
    int D;
    bool kh;
    size_t smb;
    bool xc, own;
    if (mf_plan_kh<NC>(a.rows, nsb, G, nrb, D, kh, smb, true, &xc, &own)) return FLH_ERR_UNSUPPORTED;
    if (xc) return mf_launch_d<NC, 2, false, true>(a, nrb, G, smb, s);
    if (kh) return mf_launch_d<NC, 2, true>(a, nrb, G, smb, s);
    if (own) return mf_launch_d<NC, 2, false, false, true>(a, nrb, G, smb, s);
    return D == 2 ? mf_launch_d<NC, 2, false>(a, nrb, G, smb, s) : mf_launch_d<NC, 3, false>(a, nrb, G, smb, s);
}

// Fewest columns for which STREAM_DOT takes the matrix-core kernel (measured:
// at 2 columns the streaming kernel is faster when a row's activation fits
// its registers, cols <= 4096, and slower beyond).
uint32_t mfma_min_cols(uint32_t cols) {
    return tune().mf_min_cols ? tune().mf_min_cols : (cols > 4096 ? 2u : 3u);
}

uint32_t mfma_min_cols(uint32_t cols);

template <int NC, int D, bool KH, bool OWN = false>
static int mf_moe_launch_d(const MoeArgs & a, uint32_t nrb, uint32_t gx, size_t smb, hipStream_t s) {
    if (moe_rows(a) == 0) return FLH_OK;
    if (int rc = lds_fits((const void *)k_moe_mfma<NC, D, KH, OWN>, smb, "k_moe_mfma: LDS over the limit")) return rc;
    (void)hipFuncSetAttribute((const void *)k_moe_mfma<NC, D, KH, OWN>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)smb);
    hipLaunchKernelGGL((k_moe_mfma<NC, D, KH, OWN>), dim3(gx, moe_rows(a)), dim3(MF_WAVES * 64), smb, s, a,
                       nrb | (mf_pro() << 16));
    return hip_check(hipGetLastError(), "k_moe_mfma launch");
}

template <int NC>
static int mf_moe_launch(const MoeArgs & a, hipStream_t s, bool allow_kh) {
    const uint32_t nsb = a.cols >> 8;
    // the experts that can be active at once share the CUs (one workgroup each)
    const uint32_t pairs = a.ntok * a.top_k;
    const uint32_t active = pairs < a.n_expert ? pairs : a.n_expert;
    uint32_t gx = ((uint32_t)num_cus() + active - 1) / active;
    if (gx > a.rows) gx = a.rows;
    uint32_t nrb;
    int D;
    bool kh;
    size_t smb;
    bool own;
    if (mf_plan_kh<NC>(a.rows, nsb, gx, nrb, D, kh, smb, allow_kh, nullptr, &own)) return FLH_ERR_UNSUPPORTED;
    if (kh) return mf_moe_launch_d<NC, 2, true>(a, nrb, gx, smb, s);
    if (own) return mf_moe_launch_d<NC, 2, false, true>(a, nrb, gx, smb, s);
    return D == 2 ? mf_moe_launch_d<NC, 2, false>(a, nrb, gx, smb, s) : mf_moe_launch_d<NC, 3, false>(a, nrb, gx, smb, s);
}

// Grouped Q4_K expert matvec on the matrix cores for token batches of at
// least mfma_min_cols(cols) tokens; FLH_ERR_UNSUPPORTED (nothing launched)
// otherwise or when the shape does not fit.
int launch_moe_mfma(int fmt, const MoeArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    if (fmt != FMT_Q4_K || nsb == 0 || (a.cols & 255) || nsb > 64 || a.ntok < mfma_min_cols(a.cols))
        return FLH_ERR_UNSUPPORTED;
    if (((uintptr_t)a.w & 15) || (a.estride & 15) || ((uintptr_t)a.x & 3) || (a.xstride & 3) || tune().no_mfma ||
        a.ntok * a.top_k > 256)
        return FLH_ERR_UNSUPPORTED;
    // an expert gets at most one pair per token.  K halves only as a last
    // resort: most experts get few pairs, and 4-column passes that hold the
    // whole activations beat an 8-column pass that restages them (Mixtral
    // top-2 of 8, batch 8: 217 vs 253 us)
    // 8-column passes only when an active expert averages more than 4 pairs:
    // a 4-column pass costs ~10 % less per byte, and an expert with more pairs
    // than that (rare at such averages) takes a second pass (Mixtral top-2 of
    // 8, batch 8, 2 pairs per expert on average: 209 -> 189 us)
    const uint32_t pairs = a.ntok * a.top_k, active = pairs < a.n_expert ? pairs : a.n_expert;
    const bool wide = a.ntok > 4 && (pairs + active - 1) / active > 4;
    int rc = FLH_ERR_UNSUPPORTED;
    if (wide) rc = mf_moe_launch<8>(a, s, false);
    if (rc == FLH_ERR_UNSUPPORTED) rc = mf_moe_launch<4>(a, s, false);
    if (rc == FLH_ERR_UNSUPPORTED && wide) rc = mf_moe_launch<8>(a, s, true);
    if (rc == FLH_ERR_UNSUPPORTED) rc = mf_moe_launch<4>(a, s, true);
    return rc;
}

// Q4_K x q8_K with 1..16 columns; FLH_ERR_UNSUPPORTED (nothing launched) when
// the shape does not fit (the caller then splits the columns).
int launch_dot_mfma(int fmt, const DotArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    if (fmt != FMT_Q4_K || nsb == 0 || (a.cols & 255) || nsb > 64 || a.nx < 1 || a.nx > 16)
        return FLH_ERR_UNSUPPORTED;
    if (((uintptr_t)a.w & 15) || (a.estride & 15) || ((uintptr_t)a.x & 3) || (a.xstride & 3) || tune().no_mfma)
        return FLH_ERR_UNSUPPORTED;
    if (a.nx <= 4) return mf_launch<4>(a, s);
    if (a.nx <= 8) return mf_launch<8>(a, s);
    return mf_launch<16>(a, s);
}

}  // namespace flh
