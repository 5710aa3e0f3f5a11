// flh_dot_int8.hip -- int8 STREAM_DOT kernels for gfx950 (wave64, CDNA4).
//
// Replaces the reference's GPU row-dots gdot_i8k_q4_K / gdot_i8k_q6_K /
// gdot_i8_q8_0 (src/runtime/kernels_gpu.h:307-343,535-675) and matches the
// reference CPU int8 path (src/runtime/quants.h:438-447,538-594) BIT FOR BIT:
//
//  * every integer partial (per-superblock iacc / imins, per-block idot) is
//    exact, so it may be computed by any lanes in any order;
//  * the only float work is the per-superblock (per-block for Q8_0) fmaf
//    fold into acc[t & 3] followed by (a0 + a1) + (a2 + a3).  That fold runs
//    in exactly the reference order, one lane per (row, column, accumulator).
//
// Work decomposition (one workgroup = 256 lanes = 4 waves):
//  K formats: 4 lanes per 256-weight superblock.  Lane (slot s, part c) owns
//    superblock position sb = s mod P (P = next pow2 >= superblocks per row)
//    of row-sub s / P.  Its activation slice (64 int8 of the q8_K column) is
//    loaded ONCE into registers and reused for every row the workgroup
//    streams; weights stream straight from HBM into registers (dwordx4,
//    non-temporal), two iterations in flight.  Integer partials are reduced
//    across the 4 lanes with DPP quad permutes and parked in LDS as
//    (row, column, sb) terms; after each batch of rows, lanes re-map to
//    (row, column, accumulator) and run the ordered float chains.
//  Q8_0: one lane per 34-byte block, same scheme with per-block terms.
//
// Layout facts used: Q4_K superblocks are 144 B, so with a 16-B aligned row
// every superblock is 16-B aligned.  Q6_K (210 B) and Q8_0 (34 B) blocks are
// only 2-B aligned; they are read as dword windows from the 4-B aligned
// address below and realigned with v_alignbyte (never an unaligned or
// out-of-block access).
#include "flh_common.h"
#include "flh_internal.h"
#include "flh_status.h"
#include <stdio.h>
#include <stdlib.h>

namespace flh {

__host__ __device__ inline uint32_t ceil_log2(uint32_t v) {
    uint32_t l = 0;
    while ((1u << l) < v) ++l;
    return l;
}

// ------------------------------------------------------------ Q4_K x q8_K --
struct Q4W { u32x4 h, qa, qb; };

// Lane c of a superblock loads qs[16c, 16c+16) and qs[64+16c, 64+16c+16),
// so the 4 lanes of a superblock read two contiguous 64-byte runs.  Lane c
// then owns positions l in [16(c&1), 16(c&1)+16) of groups
// g0 = 2(c>>1), g0+1 (low/high nibbles of the first run) and g0+4, g0+5
// (second run).
__device__ __forceinline__ Q4W q4_load(const uint8_t * blk, uint32_t c) {
    Q4W r;
    r.h  = ld4_nt(blk);
    r.qa = ld4_nt(blk + 16 + 16 * c);
    r.qb = ld4_nt(blk + 80 + 16 * c);
    return r;
}

template <int NX>
struct Q4X {                    // activation slice of one lane, NX columns
    int q[NX][4][4];            // [column][group slot][dword]: x[32g + 16(c&1) ..+16)
    int bs[NX][4];              // bsums[2g + (c&1)] of the lane's 4 groups
};

template <int NX>
__device__ __forceinline__ void q4x_load(Q4X<NX> & X, const uint8_t * const * xk,
                                         uint32_t nx, uint32_t sb, uint32_t c) {
    const uint32_t g0 = 2 * (c >> 1), h = c & 1;
    const uint32_t gs[4] = {g0, g0 + 1, g0 + 4, g0 + 5};
#pragma unroll
    for (int p = 0; p < NX; ++p) {
        const uint8_t * b = xk[p < (int)nx ? p : 0] + (size_t)sb * 292;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32x4 v = ld4(b + 36 + 32 * gs[k] + 16 * h);
            X.q[p][k][0] = v.x; X.q[p][k][1] = v.y; X.q[p][k][2] = v.z; X.q[p][k][3] = v.w;
            X.bs[p][k] = (int)*(const int16_t *)(b + 4 + 2 * (2 * gs[k] + h));
        }
    }
}

// ------------------------------------------------------------ Q6_K x q8_K --
struct Q6W { u32x4 a, b, h, s; uint32_t a4, b4, h4, s4, sh; };

__device__ __forceinline__ Q6W q6_load(const uint8_t * blk, uint32_t c) {
    const uint32_t hh = c >> 1, bb = c & 1;
    const uintptr_t ba = (uintptr_t)blk;
    const uint8_t * f = (const uint8_t *)(ba & ~(uintptr_t)3);
    Q6W r;
    r.sh = (uint32_t)(ba & 3);
    const uint32_t oa = 64 * hh + 16 * bb, ob = oa + 32, oh = 128 + 32 * hh + 16 * bb;
    r.a = ld4_nt(f + oa); r.a4 = ld1(f + oa + 16);
    r.b = ld4_nt(f + ob); r.b4 = ld1(f + ob + 16);
    r.h = ld4_nt(f + oh); r.h4 = ld1(f + oh + 16);
    r.s = ld4(f + 192);
    r.s4 = ldh(f + 208) | (ldh(blk + 208) << 16);
    return r;
}

template <int NX>
struct Q6X {
    int q[NX][4][4];            // [column][group g][dword i]
    int b32[NX][4];             // 32 * bsums[8h + 2g + b]
};

template <int NX>
__device__ __forceinline__ void q6x_load(Q6X<NX> & X, const uint8_t * const * xk,
                                         uint32_t nx, uint32_t sb, uint32_t c) {
    const uint32_t hh = c >> 1, bb = c & 1;
#pragma unroll
    for (int p = 0; p < NX; ++p) {
        const uint8_t * b = xk[p < (int)nx ? p : 0] + (size_t)sb * 292;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const u32x4 v = ld4(b + 36 + 128 * hh + 32 * g + 16 * bb);
            X.q[p][g][0] = v.x; X.q[p][g][1] = v.y; X.q[p][g][2] = v.z; X.q[p][g][3] = v.w;
            X.b32[p][g] = 32 * (int)*(const int16_t *)(b + 4 + 2 * (8 * hh + 2 * g + bb));
        }
    }
}

// ------------------------------------------------------ K-format kernel core --
// smem layout (ints): TI[nr][NX][P] (+ TM[nr][NX][P] for Q4_K), TH[nr][P],
// XD[NX][P] (float, q8_K d of each column/superblock).
template <int FMT>
__host__ __device__ inline size_t kq_smem_bytes(uint32_t nr, uint32_t nx_t, uint32_t P) {
    const size_t terms = (size_t)nr * nx_t * P * (FMT == FMT_Q4_K ? 2 : 1);
    return 4 * (terms + (size_t)nr * P + (size_t)nx_t * P);
}

template <int FMT, int NX, int D>
__device__ __forceinline__ void kq_core(const uint8_t * __restrict__ w, uint32_t rows,
                                        uint32_t cols, const uint8_t * const * xk,
                                        float * const * yc, uint32_t nx, uint32_t nr,
                                        uint32_t batch0, uint32_t bstep, int * smem) {
    constexpr uint32_t BLK = FMT == FMT_Q4_K ? 144 : 210;
    const uint32_t nsb = cols >> 8;
    const uint32_t lgP = ceil_log2(nsb), P = 1u << lgP;
    const uint32_t rpi = 64u >> lgP;
    const uint64_t rb = (uint64_t)nsb * BLK;
    const uint32_t tid = threadIdx.x, c = tid & 3, slot = tid >> 2;
    const uint32_t rsub = slot >> lgP, sbl = slot & (P - 1);
    const bool act = sbl < nsb;
    const uint32_t sb = act ? sbl : nsb - 1;

    int * TI = smem;
    int * TM = TI + (size_t)nr * NX * P;
    uint32_t * TH = (uint32_t *)(FMT == FMT_Q4_K ? TM + (size_t)nr * NX * P : TM);
    float * XD = (float *)(TH + (size_t)nr * P);

    for (uint32_t i = tid; i < NX * P; i += 256) {
        const uint32_t p = i >> lgP, q = i & (P - 1);
        XD[i] = (p < nx && q < nsb) ? *(const float *)(xk[p] + (size_t)q * 292) : 0.f;
    }

    // per-lane activation slice, resident for the whole launch
    typename std::conditional<FMT == FMT_Q4_K, Q4X<NX>, Q6X<NX>>::type X;
    if constexpr (FMT == FMT_Q4_K) q4x_load<NX>(X, xk, nx, sb, c);
    else                           q6x_load<NX>(X, xk, nx, sb, c);

    using WT = typename std::conditional<FMT == FMT_Q4_K, Q4W, Q6W>::type;
    auto wload = [&](uint32_t row) -> WT {
        const uint8_t * blk = w + (size_t)row * rb + (size_t)sb * BLK;
        if constexpr (FMT == FMT_Q4_K) return q4_load(blk, c);
        else                           return q6_load(blk, c);
    };

    // integer partials of one (row-sub, superblock, part) item -> LDS terms
    auto process = [&](const WT & Wv, uint32_t rl, uint32_t nrow) {
        const bool wr = act && c == 0 && rl < nrow;
        if constexpr (FMT == FMT_Q4_K) {
            const Q4W & W = Wv;
            // 6-bit scale/min unpack for all 8 groups, packed one byte per group
            const uint32_t sclo = W.h.y & 0x3F3F3F3Fu;
            const uint32_t mlo  = W.h.z & 0x3F3F3F3Fu;
            const uint32_t schi = (W.h.w & 0x0F0F0F0Fu) | ((W.h.y >> 2) & 0x30303030u);
            const uint32_t mhi  = ((W.h.w >> 4) & 0x0F0F0F0Fu) | ((W.h.z >> 2) & 0x30303030u);
            const uint32_t sh = (c >> 1) * 16;
            const int sc[4] = {(int)((sclo >> sh) & 0xFF), (int)((sclo >> (sh + 8)) & 0xFF),
                               (int)((schi >> sh) & 0xFF), (int)((schi >> (sh + 8)) & 0xFF)};
            const int mn[4] = {(int)((mlo >> sh) & 0xFF), (int)((mlo >> (sh + 8)) & 0xFF),
                               (int)((mhi >> sh) & 0xFF), (int)((mhi >> (sh + 8)) & 0xFF)};
            const uint32_t q[2][4] = {{W.qa.x, W.qa.y, W.qa.z, W.qa.w},
                                      {W.qb.x, W.qb.y, W.qb.z, W.qb.w}};
            int nib[4][4];          // [group slot][dword]
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                nib[0][k] = (int)(q[0][k] & 0x0F0F0F0Fu);
                nib[1][k] = (int)((q[0][k] >> 4) & 0x0F0F0F0Fu);
                nib[2][k] = (int)(q[1][k] & 0x0F0F0F0Fu);
                nib[3][k] = (int)((q[1][k] >> 4) & 0x0F0F0F0Fu);
            }
#pragma unroll
            for (int p = 0; p < NX; ++p) {
                int ia = 0, im = 0;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    int d = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) d = dot4(nib[g][k], X.q[p][g][k], d);
                    ia += sc[g] * d;
                    im += mn[g] * X.bs[p][g];
                }
                ia += qx1(ia); ia += qx2(ia);
                im += qx1(im); im += qx2(im);
                if (wr && p < (int)nx) {
                    TI[((rl * NX + p) << lgP) + sb] = ia;
                    TM[((rl * NX + p) << lgP) + sb] = im;
                }
            }
            if (wr) TH[(rl << lgP) + sb] = W.h.x;
        } else {
            const Q6W & W = Wv;
            const uint32_t sh = W.sh;
            const uint32_t A[5] = {W.a.x, W.a.y, W.a.z, W.a.w, W.a4};
            const uint32_t B[5] = {W.b.x, W.b.y, W.b.z, W.b.w, W.b4};
            const uint32_t H[5] = {W.h.x, W.h.y, W.h.z, W.h.w, W.h4};
            const uint32_t S[5] = {W.s.x, W.s.y, W.s.z, W.s.w, W.s4};
            uint32_t Sa[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) Sa[i] = alignb(S[i + 1], S[i], sh);
            const uint32_t dbits = alignb(W.s4, W.s4, sh) & 0xFFFFu;
            const uint32_t hh = c >> 1, bb = c & 1;
            const uint32_t sd0 = hh ? Sa[2] : Sa[0], sd1 = hh ? Sa[3] : Sa[1];
            const int sc[4] = {(int)(int8_t)(sd0 >> (8 * bb)), (int)(int8_t)(sd0 >> (8 * bb + 16)),
                               (int)(int8_t)(sd1 >> (8 * bb)), (int)(int8_t)(sd1 >> (8 * bb + 16))};
            int g[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t a = alignb(A[i + 1], A[i], sh);
                const uint32_t b = alignb(B[i + 1], B[i], sh);
                const uint32_t h = alignb(H[i + 1], H[i], sh);
                g[0][i] = (int)((a & 0x0F0F0F0Fu) | ((h & 0x03030303u) << 4));
                g[1][i] = (int)((b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u));
                g[2][i] = (int)(((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u));
                g[3][i] = (int)(((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u));
            }
#pragma unroll
            for (int p = 0; p < NX; ++p) {
                int ia = 0;
#pragma unroll
                for (int gg = 0; gg < 4; ++gg) {
                    int d = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) d = dot4(g[gg][i], X.q[p][gg][i], d);
                    ia += sc[gg] * (d - X.b32[p][gg]);
                }
                ia += qx1(ia); ia += qx2(ia);
                if (wr && p < (int)nx) TI[((rl * NX + p) << lgP) + sb] = ia;
            }
            if (wr) TH[(rl << lgP) + sb] = dbits;
        }
    };

    const uint32_t nbatch = (rows + nr - 1) / nr;
    const uint32_t nit = (nr + rpi - 1) / rpi;
    const uint32_t fk = tid & 3, fp = (tid >> 2) % NX, frl = tid / (4 * NX);
    for (uint32_t bt = batch0; bt < nbatch; bt += bstep) {
        const uint32_t row0 = bt * nr;
        const uint32_t nrow = min(nr, rows - row0);
        auto clamp_row = [&](uint32_t rl) { return row0 + (rl < nrow ? rl : nrow - 1); };
        // The fold lane's y value, fetched before the weight stream starts.
        // Every load in this loop nest is unconditional (addresses clamped
        // to valid rows) so the compiler can count outstanding loads
        // statically and keep D iterations in flight; a conditional load
        // makes it fall back to waiting for all of them.
        const bool fok = frl < nrow && fp < nx;
        const float yold = yc[fp][row0 + (frl < nrow ? frl : nrow - 1)];
        WT buf[D];
#pragma unroll
        for (int j = 0; j < D; ++j) buf[j] = wload(clamp_row(j * rpi + rsub));
        for (uint32_t it0 = 0; it0 < nit; it0 += D) {
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const uint32_t it = it0 + j;
                process(buf[j], it * rpi + rsub, nrow);     // writes nothing past nrow
                buf[j] = wload(clamp_row((it + D) * rpi + rsub));
            }
        }
        __syncthreads();
        // ordered float fold: lane -> (row, column, accumulator k)
        {
            const uint32_t k = fk, p = fp, rl = frl;
            const bool ok = fok;
            float acc = 0.f;
            if (ok) {
                const int * ti = TI + ((rl * NX + p) << lgP);
                const int * tm = TM + ((rl * NX + p) << lgP);
                const uint32_t * th = TH + (rl << lgP);
                const float * xd = XD + (p << lgP);
                for (uint32_t s = k; s < nsb; s += 4) {
                    const float dk = xd[s];
                    if constexpr (FMT == FMT_Q4_K) {
                        const float d = h2f(th[s] & 0xFFFFu), dmin = h2f(th[s] >> 16);
                        acc = fmaf(d * dk, (float)ti[s], acc);
                        acc = fmaf(-(dmin * dk), (float)tm[s], acc);
                    } else {
                        const float d = h2f(th[s]);
                        acc = fmaf(d * dk, (float)ti[s], acc);
                    }
                }
            }
            const float s01 = acc + qx1f(acc);          // lane k=0: a0+a1, k=2: a2+a3
            const float r = s01 + qx2f(s01);            // lane k=0: (a0+a1)+(a2+a3)
            if (ok && k == 0) yc[p][row0 + rl] = yold + r;
        }
        __syncthreads();
    }
}

template <int FMT, int NX, int D>
__global__ __launch_bounds__(256) void k_dot_i8k(DotArgs a, uint32_t nr) {
    extern __shared__ int smem[];
    const uint8_t * w = a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0);
    const uint8_t * xk[NX];
    float * yc[NX];
#pragma unroll
    for (int p = 0; p < NX; ++p) {
        const uint32_t pp = p < (int)a.nx ? p : 0;
        xk[p] = (const uint8_t *)(a.x + (size_t)pp * a.xstride) + xqk_off(a.cols);
        yc[p] = a.y + (size_t)pp * a.ystride;
    }
    kq_core<FMT, NX, D>(w, a.rows, a.cols, xk, yc, a.nx, nr, blockIdx.x, gridDim.x, smem);
}

// Grouped expert kernel: blockIdx.y = expert.  The workgroup scans the
// routing table for its expert; with no routed (token, slot) pair it exits
// before touching a weight byte.  Columns are processed NX at a time.
template <int FMT, int NX>
__global__ __launch_bounds__(256) void k_moe_i8k(MoeArgs a, uint32_t nr) {
    extern __shared__ int smem[];
    __shared__ uint32_t cols_s[256];
    __shared__ uint32_t ncols_s;
    const uint32_t e = blockIdx.y;
    if (threadIdx.x == 0) {
        uint32_t n = 0;
        for (uint32_t i = 0; i < a.ntok * a.top_k && n < 256; ++i)
            if (a.ids[i] == e) cols_s[n++] = i;          // i = tok*top_k + slot
        ncols_s = n;
    }
    __syncthreads();
    const uint32_t ncols = ncols_s;
    if (ncols == 0) return;
    const uint8_t * w = a.w + (size_t)e * a.estride;
    for (uint32_t p0 = 0; p0 < ncols; p0 += NX) {
        const uint32_t nx = min((uint32_t)NX, ncols - p0);
        const uint8_t * xk[NX];
        float * yc[NX];
#pragma unroll
        for (int p = 0; p < NX; ++p) {
            const uint32_t ts = cols_s[p0 + (p < (int)nx ? p : 0)];
            const uint32_t xi = a.x_per_slot ? ts : ts / a.top_k;
            xk[p] = (const uint8_t *)(a.x + (size_t)xi * a.xstride) + xqk_off(a.cols);
            yc[p] = a.y + (size_t)ts * a.ystride;
        }
        kq_core<FMT, NX, 2>(w, a.rows, a.cols, xk, yc, nx, nr, blockIdx.x, gridDim.x, smem);
        __syncthreads();
    }
}

// ----------------------------------------------------- Q8_0 / Q5_0 x q8_1 --
// One lane per 32-weight block (Q5_0: 5-bit values built in registers, the
// -16 offset applied as 16 x the block's activation sum, fl_dot_i8_q5_0,
// src/runtime/quants.h:449-466); NK blocks per lane (row of up to 256*NK
// blocks).  Terms: idot per (row, column, block) and the weight scale bits
// per (row, block); chain acc[b & 3] = fmaf(dw * dx, idot, .).
// terms, weight scales, activation scales, then the IQ codebook (2 KiB)
__host__ __device__ inline size_t q8_smem_bytes(uint32_t nr, uint32_t nx_t, uint32_t P) {
    return 4 * ((size_t)nr * nx_t * P + (size_t)nr * P + (size_t)nx_t * P) + 2048;
}

template <int FMT, int NX, int NK>
__global__ __launch_bounds__(256) void k_dot_i8_b32(DotArgs a, uint32_t nr) {
    extern __shared__ int smem[];
    const uint8_t * w = a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0);
    const uint32_t nb = a.cols >> 5;
    const uint32_t lgP = ceil_log2(nb), P = 1u << lgP;   // P <= 256*NK
    const uint32_t rpi = NK == 1 ? (256u >> lgP) : 1u;
    constexpr bool IQ = FMT == FMT_IQ2_XXS || FMT == FMT_IQ3_XXS;
    // block bytes (IQ: of a 256-element superblock holding 8 groups)
    constexpr uint32_t BB = FMT == FMT_Q5_0 ? 22 : FMT == FMT_Q8_0 ? 34 : iq_block_bytes(FMT);
    const uint64_t rb = IQ ? (uint64_t)(nb >> 3) * BB : (uint64_t)nb * BB;
    const uint32_t tid = threadIdx.x;
    const uint32_t rsub = NK == 1 ? (tid >> lgP) : 0u;
    uint32_t bl[NK];
    bool act[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        const uint32_t b = NK == 1 ? (tid & (P - 1)) : tid + 256u * k;
        act[k] = b < nb;
        bl[k] = act[k] ? b : nb - 1;
    }
    int * TI = smem;
    uint32_t * TH = (uint32_t *)(TI + (size_t)nr * NX * P);
    float * XD = (float *)(TH + (size_t)nr * P);
    uint32_t * GR = (uint32_t *)(XD + (size_t)NX * P);   // IQ codebook, 2 KiB
    if constexpr (FMT == FMT_IQ2_XXS) {
        GR[2 * tid] = (uint32_t)k_iq2_grid[tid];
        GR[2 * tid + 1] = (uint32_t)(k_iq2_grid[tid] >> 32);
    } else if constexpr (FMT == FMT_IQ3_XXS) {
        GR[tid] = k_iq3_grid[tid];
    }
    if constexpr (IQ) __syncthreads();

    const uint8_t * xq[NX];
#pragma unroll
    for (int p = 0; p < NX; ++p) {
        const uint32_t pp = p < (int)a.nx ? p : 0;
        xq[p] = (const uint8_t *)(a.x + (size_t)pp * a.xstride) + xq_off(a.cols);
    }
    for (uint32_t i = tid; i < NX * P; i += 256) {
        const uint32_t p = i >> lgP, q = i & (P - 1);
        XD[i] = (p < a.nx && q < nb) ? h2f(ldh(xq[p] + (size_t)q * 36)) : 0.f;
    }
    int X[NX][NK][8];
#pragma unroll
    for (int p = 0; p < NX; ++p)
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const uint8_t * b = xq[p] + (size_t)bl[k] * 36 + 4;
            const u32x4 v0 = ld4(b), v1 = ld4(b + 16);
            X[p][k][0] = v0.x; X[p][k][1] = v0.y; X[p][k][2] = v0.z; X[p][k][3] = v0.w;
            X[p][k][4] = v1.x; X[p][k][5] = v1.y; X[p][k][6] = v1.z; X[p][k][7] = v1.w;
        }
    // Q5_0: the block's activation sum (the -16 offset term), exact
    int XS[NX][NK];
#pragma unroll
    for (int p = 0; p < NX; ++p)
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            int t = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) t = dot4(0x01010101, X[p][k][j], t);
            XS[p][k] = t;
        }

    // A block's bytes from the dword-aligned window at f (blocks are 2-byte
    // aligned; nothing past the block's last byte is read).
    struct W8 { u32x4 d0, d1; uint32_t d8, sh; };
    auto wload = [&](uint32_t row, uint32_t b) -> W8 {
        if constexpr (IQ) {
            // group b = (superblock b/8, group b%8); 2-byte aligned pieces:
            // d, the 8 index bytes (IQ2: 4 indices + w1), IQ3's w1 word
            const uint8_t * sbp = w + (size_t)row * rb + (size_t)(b >> 3) * BB;
            const uint8_t * q = sbp + 2 + 8 * (b & 7);
            const uintptr_t qa = (uintptr_t)q;
            const uint8_t * f = (const uint8_t *)(qa & ~(uintptr_t)3);
            W8 r;
            r.sh = (uint32_t)(qa & 3);
            const uint32_t A = *(const uint32_t *)f, B = *(const uint32_t *)(f + 4);
            const uint32_t Cw = r.sh ? ldh(f + 8) : 0u;
            r.d0 = u32x4{alignb(B, A, r.sh), alignb(Cw, B, r.sh), ldh(sbp), 0u};
            if constexpr (FMT == FMT_IQ3_XXS) {
                const uint8_t * sw = sbp + 66 + 4 * (b & 7);
                r.d0.w = ldh(sw) | (ldh(sw + 2) << 16);
            }
            r.d1 = u32x4{0u, 0u, 0u, 0u};
            r.d8 = 0;
            return r;
        }
        const uint8_t * blk = w + (size_t)row * rb + (size_t)b * BB;
        const uintptr_t ba = (uintptr_t)blk;
        const uint8_t * f = (const uint8_t *)(ba & ~(uintptr_t)3);
        W8 r;
        r.sh = (uint32_t)(ba & 3);
        r.d0 = ld4_nt(f);
        if constexpr (FMT == FMT_Q5_0) {
            r.d1 = u32x4{*(const uint32_t *)(f + 16), r.sh ? *(const uint32_t *)(f + 20) : ldh(f + 20), 0u, 0u};
            r.d8 = 0;
        } else {
            r.d1 = ld4_nt(f + 16);
            r.d8 = ldh(f + 32) | (ldh(blk + 32) << 16);
        }
        return r;
    };

    const uint32_t nbatch = (a.rows + nr - 1) / nr;
    const uint32_t nit = (nr + rpi - 1) / rpi;
    for (uint32_t bt = blockIdx.x; bt < nbatch; bt += gridDim.x) {
        const uint32_t row0 = bt * nr, nrow = min(nr, a.rows - row0);
        auto clamp_row = [&](uint32_t rl) { return row0 + (rl < nrow ? rl : nrow - 1); };
        W8 cur[NK];
#pragma unroll
        for (int k = 0; k < NK; ++k) cur[k] = wload(clamp_row(rsub), bl[k]);
        for (uint32_t it = 0; it < nit; ++it) {
            W8 nxt[NK];
#pragma unroll
            for (int k = 0; k < NK; ++k) nxt[k] = cur[k];
            if (it + 1 < nit) {
#pragma unroll
                for (int k = 0; k < NK; ++k) nxt[k] = wload(clamp_row((it + 1) * rpi + rsub), bl[k]);
            }
            const uint32_t rl = it * rpi + rsub;
#pragma unroll
            for (int k = 0; k < NK; ++k) {
                const W8 & W = cur[k];
                const bool wr = act[k] && rl < nrow && rl < nr;
                uint32_t dbits;
                int qs[8];
                if constexpr (IQ) {
                    // signed grid magnitudes of the group's 32 elements,
                    // dword j = elements 4j..4j+3 (quants.h:237-290)
                    const uint32_t w0 = W.d0.x;
                    const uint32_t w1 = FMT == FMT_IQ2_XXS ? W.d0.y : W.d0.w;
#pragma unroll
                    for (int l = 0; l < 4; ++l) {
                        const uint32_t sg = iq_sign8(w1 >> (7 * l));
                        uint32_t lo, hi;
                        if constexpr (FMT == FMT_IQ2_XXS) {
                            const uint32_t gi = (w0 >> (8 * l)) & 0xFFu;
                            lo = GR[2 * gi];
                            hi = GR[2 * gi + 1];
                        } else {
                            const uint32_t ix = l < 2 ? w0 : W.d0.y;
                            lo = GR[(ix >> (16 * (l & 1))) & 0xFFu];
                            hi = GR[(ix >> (16 * (l & 1) + 8)) & 0xFFu];
                        }
                        qs[2 * l] = (int)iq_apply(lo, iq_neg4(sg));
                        qs[2 * l + 1] = (int)iq_apply(hi, iq_neg4(sg >> 4));
                    }
                    dbits = __float_as_uint(iq_db(FMT, h2f(W.d0.z), w1));
                } else if constexpr (FMT == FMT_Q5_0) {
                    // E = the block's bytes 0..21; d, qh, then 16 bytes of nibble pairs
                    const uint32_t D[6] = {W.d0.x, W.d0.y, W.d0.z, W.d0.w, W.d1.x, W.d1.y};
                    uint32_t E[6];
#pragma unroll
                    for (int i = 0; i < 5; ++i) E[i] = alignb(D[i + 1], D[i], W.sh);
                    E[5] = D[5] >> (8 * W.sh);
                    dbits = E[0] & 0xFFFFu;
                    const uint32_t qh = (E[0] >> 16) | (E[1] << 16);
#pragma unroll
                    for (int k4 = 0; k4 < 4; ++k4) {
                        const uint32_t q = alignb(E[2 + k4], E[1 + k4], 2);
                        qs[k4] = (int)((q & 0x0F0F0F0Fu) | (spread4((qh >> (4 * k4)) & 0xFu) << 4));
                        qs[4 + k4] = (int)(((q >> 4) & 0x0F0F0F0Fu) | (spread4((qh >> (16 + 4 * k4)) & 0xFu) << 4));
                    }
                } else {
                    const uint32_t D[9] = {W.d0.x, W.d0.y, W.d0.z, W.d0.w,
                                           W.d1.x, W.d1.y, W.d1.z, W.d1.w, W.d8};
                    dbits = W.sh ? (D[0] >> 16) : (D[0] & 0xFFFFu);
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        qs[j] = (int)(W.sh ? D[j + 1] : alignb(D[j + 1], D[j], 2));
                }
#pragma unroll
                for (int p = 0; p < NX; ++p) {
                    int d = 0;
#pragma unroll
                    for (int j = 0; j < 8; ++j) d = dot4(qs[j], X[p][k][j], d);
                    if constexpr (FMT == FMT_Q5_0) d -= 16 * XS[p][k];     // (idot - 16 isum), quants.h:449-466
                    if (wr && p < (int)a.nx) TI[((rl * NX + p) << lgP) + bl[k]] = d;
                }
                if (wr) TH[(rl << lgP) + bl[k]] = dbits;
            }
#pragma unroll
            for (int k = 0; k < NK; ++k) cur[k] = nxt[k];
        }
        __syncthreads();
        for (uint32_t base = 0; base < nr * NX * 4; base += 256) {
            const uint32_t t = base + tid;
            const uint32_t k = t & 3, p = (t >> 2) % NX, rl = t / (4 * NX);
            const bool ok = rl < nrow && p < a.nx;
            float acc = 0.f;
            if (ok) {
                const int * ti = TI + ((rl * NX + p) << lgP);
                const uint32_t * th = TH + (rl << lgP);
                const float * xd = XD + (p << lgP);
                for (uint32_t b = k; b < nb; b += 4) {
                    const float ws = IQ ? __uint_as_float(th[b]) : h2f(th[b]);
                    acc = fmaf(ws * xd[b], (float)ti[b], acc);
                }
            }
            const float s01 = acc + qx1f(acc);
            const float r = s01 + qx2f(s01);
            if (ok && k == 0) {
                float * yp = a.y + (size_t)p * a.ystride + row0 + rl;
                *yp = *yp + r;
            }
        }
        __syncthreads();
    }
}

// ----------------------------------------------------------------- launch --
// Launch shape of the K-format kernels: a persistent grid of at most
// wgs_per_cu workgroups per CU, each looping over batches of nr rows with a
// D-deep weight pipeline.  FLH_KQ_TUNE="wgs_per_cu,nr,D" overrides the
// defaults (development sweeps only).
struct KqTune { uint32_t wgs_per_cu, nr, D; };
static KqTune kq_tune() { return KqTune{tune().kq_wgs_per_cu, tune().kq_nr, tune().kq_D}; }

static uint32_t pick_nr(uint32_t rows, uint32_t rpi, uint32_t nr_max) {
    const uint32_t target = (uint32_t)num_cus() * 8u;
    uint32_t nr = (rows + target - 1) / target;
    if (nr < 1) nr = 1;
    if (nr > nr_max) nr = nr_max;
    if (nr > rpi) nr = (nr / rpi) * rpi;
    return nr;
}

template <int FMT, int NX, int D>
static int launch_kq_d(const DotArgs & a, uint32_t nr, uint32_t grid, size_t sm, hipStream_t s) {
    hipLaunchKernelGGL((k_dot_i8k<FMT, NX, D>), dim3(grid), dim3(256), sm, s, a, nr);
    return hip_check(hipGetLastError(), "k_dot_i8k launch");
}

template <int FMT, int NX>
static int launch_kq(const DotArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    const uint32_t P = 1u << ceil_log2(nsb), rpi = 64u / P;
    const KqTune t = kq_tune();
    uint32_t nr;
    if (t.nr) {
        nr = t.nr > 64u / NX ? 64u / NX : t.nr;
        if (nr > rpi) nr = (nr / rpi) * rpi;
    } else {
        nr = pick_nr(a.rows, rpi, 64u / NX);
    }
    const size_t sm = kq_smem_bytes<FMT>(nr, NX, P);
    const uint32_t nbatch = (a.rows + nr - 1) / nr;
    const uint32_t cap = (uint32_t)num_cus() * (t.wgs_per_cu ? t.wgs_per_cu : 4u);
    const uint32_t grid = nbatch < cap ? nbatch : cap;
    switch (t.D) {
        case 1: return launch_kq_d<FMT, NX, 1>(a, nr, grid, sm, s);
        case 4: return launch_kq_d<FMT, NX, 4>(a, nr, grid, sm, s);
        default: return launch_kq_d<FMT, NX, 2>(a, nr, grid, sm, s);
    }
}

int launch_dot_i8k(int fmt, const DotArgs & a0, hipStream_t s) {
    const uint32_t nsb = a0.cols >> 8;
    if (nsb == 0 || nsb > 64 || (a0.cols & 255))
        return set_error(FLH_ERR_UNSUPPORTED, "i8k dot: cols must be a multiple of 256, <= 16384");
    if (a0.rows == 0 || a0.nx == 0) return FLH_OK;
    // several Q4_K columns: the int8 matrix-core kernel, all columns in one
    // pass when they fit its LDS plan, else in groups of 8 or 4
    if (fmt == FMT_Q4_K && a0.nx >= mfma_min_cols(a0.cols)) {
        for (uint32_t gs : {16u, 8u, 4u}) {
            if (gs < 16 && a0.nx <= gs) continue;
            int rc = FLH_OK;
            for (uint32_t p0 = 0; p0 < a0.nx && rc == FLH_OK; p0 += gs) {
                DotArgs a = a0;
                a.nx = a0.nx - p0 < gs ? a0.nx - p0 : gs;
                a.x = a0.x + (size_t)p0 * a0.xstride;
                a.y = a0.y + (size_t)p0 * a0.ystride;
                rc = launch_dot_mfma(fmt, a, s);
                // the plan depends on the column count only through NC, so a
                // later (narrower) group never fails where the first fitted
                if (rc == FLH_ERR_UNSUPPORTED && p0 != 0) return set_error(rc, "mfma dot: group plan");
            }
            if (rc != FLH_ERR_UNSUPPORTED) return rc;
        }
    }
    for (uint32_t p0 = 0, g = 4; p0 < a0.nx; p0 += g) {
        DotArgs a = a0;
        int rc = FLH_ERR_UNSUPPORTED;
        // 5-8 columns of matrices of 12288 rows or more on the matrix cores
        // (14336x4096, 8 columns: 26.6 -> 21.8 us; 6144 rows: 14.6 against
        // 16.8 us, too few tiles); at 2-4 columns the streaming kernel is as
        // fast or faster
        if (fmt == FMT_Q6_K && a0.nx - p0 >= 2 && a0.nx - p0 >= tune().q6mf_cols &&
            a0.rows >= tune().q6mf_rows && !tune().no_q6mf) {
            a.x = a0.x + (size_t)p0 * a0.xstride;
            a.y = a0.y + (size_t)p0 * a0.ystride;
            a.nx = a0.nx - p0 < 16 ? a0.nx - p0 : 16;               // 9-16 columns in one pass where it fits
            rc = a.nx > 8 ? launch_dot_q6mf(a, s) : FLH_ERR_UNSUPPORTED;
            if (rc == FLH_ERR_UNSUPPORTED) {
                a.nx = a0.nx - p0 < 8 ? a0.nx - p0 : 8;
                rc = launch_dot_q6mf(a, s);
            }
            if (rc != FLH_ERR_UNSUPPORTED) {
                if (rc) return rc;
                g = a.nx;
                continue;
            }
        }
        if (fmt == FMT_Q6_K && a0.nx - p0 > 4) {                  // 5-8 columns in one streaming pass
            a.nx = a0.nx - p0 < 8 ? a0.nx - p0 : 8;
            a.x = a0.x + (size_t)p0 * a0.xstride;
            a.y = a0.y + (size_t)p0 * a0.ystride;
            rc = launch_dot_kstream(fmt, a, s);
            if (rc != FLH_ERR_UNSUPPORTED) {
                if (rc) return rc;
                g = a.nx;
                continue;
            }
        }
        g = 4;
        a.nx = a0.nx - p0 < 4 ? a0.nx - p0 : 4;
        a.x = a0.x + (size_t)p0 * a0.xstride;
        a.y = a0.y + (size_t)p0 * a0.ystride;
        rc = launch_dot_kstream(fmt, a, s);
        if (rc != FLH_ERR_UNSUPPORTED) {
            if (rc) return rc;
            continue;
        }
        if (fmt == FMT_Q4_K) {
            rc = a.nx == 1 ? launch_kq<FMT_Q4_K, 1>(a, s)
               : a.nx == 2 ? launch_kq<FMT_Q4_K, 2>(a, s) : launch_kq<FMT_Q4_K, 4>(a, s);
        } else if (fmt == FMT_Q6_K) {
            rc = a.nx == 1 ? launch_kq<FMT_Q6_K, 1>(a, s)
               : a.nx == 2 ? launch_kq<FMT_Q6_K, 2>(a, s) : launch_kq<FMT_Q6_K, 4>(a, s);
        } else {
            return set_error(FLH_ERR_UNSUPPORTED, "i8k dot: format has no q8_K path");
        }
        if (rc) return rc;
    }
    return FLH_OK;
}

template <int FMT, int NX>
static int launch_moe_t(const MoeArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    const uint32_t P = 1u << ceil_log2(nsb), rpi = 64u / P;
    // experts split the chip: aim for ~8 workgroups per CU over all experts
    uint32_t nr = (uint32_t)(((uint64_t)a.rows * a.n_expert + num_cus() * 8u - 1) / (num_cus() * 8u));
    if (nr < 1) nr = 1;
    if (nr > 64u / NX) nr = 64u / NX;
    if (nr > rpi) nr = (nr / rpi) * rpi;
    const size_t sm = kq_smem_bytes<FMT>(nr, NX, P);
    const uint32_t grid = (a.rows + nr - 1) / nr;
    hipLaunchKernelGGL((k_moe_i8k<FMT, NX>), dim3(grid, a.n_expert), dim3(256), sm, s, a, nr);
    return hip_check(hipGetLastError(), "k_moe_i8k launch");
}

int launch_moe_i8k(int fmt, const MoeArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    if (nsb == 0 || nsb > 64 || (a.cols & 255))
        return set_error(FLH_ERR_UNSUPPORTED, "moe i8k: cols must be a multiple of 256, <= 16384");
    if (a.rows == 0 || a.ntok == 0 || a.top_k == 0) return FLH_OK;
    if (a.ntok * a.top_k > 256) return set_error(FLH_ERR_UNSUPPORTED, "moe: ntok*top_k > 256");
    int rc = FLH_ERR_UNSUPPORTED;
    if (a.ntok == 1 && tune().sbl) rc = launch_moe_sbl(fmt, a, s);     // one token: superblock per lane
    if (rc != FLH_ERR_UNSUPPORTED) return rc;
    rc = launch_moe_mfma(fmt, a, s);
    if (rc != FLH_ERR_UNSUPPORTED) return rc;
    rc = launch_moe_kstream(fmt, a, s);
    if (rc != FLH_ERR_UNSUPPORTED) return rc;
    if (fmt == FMT_Q4_K) return launch_moe_t<FMT_Q4_K, 4>(a, s);
    if (fmt == FMT_Q6_K) return launch_moe_t<FMT_Q6_K, 4>(a, s);
    return set_error(FLH_ERR_UNSUPPORTED, "moe i8k: format has no q8_K path");
}

template <int FMT, int NX, int NK>
static int launch_q8(const DotArgs & a, hipStream_t s) {
    const uint32_t nb = a.cols >> 5;
    const uint32_t P = 1u << ceil_log2(nb);
    const uint32_t rpi = NK == 1 ? 256u / P : 1u;
    // LDS budget 48 KiB for the terms
    uint32_t nr_max = 64u / NX;
    while (nr_max > 1 && q8_smem_bytes(nr_max, NX, P) > 48u * 1024u) nr_max >>= 1;
    const uint32_t nr = pick_nr(a.rows, rpi, nr_max);
    const size_t sm = q8_smem_bytes(nr, NX, P);
    const uint32_t grid = (a.rows + nr - 1) / nr;
    hipLaunchKernelGGL((k_dot_i8_b32<FMT, NX, NK>), dim3(grid), dim3(256), sm, s, a, nr);
    return hip_check(hipGetLastError(), "k_dot_i8_b32 launch");
}

template <int FMT>
static int launch_i8_b32(const DotArgs & a0, hipStream_t s) {
    const uint32_t nb = a0.cols >> 5;
    if (nb == 0 || nb > 512 || (a0.cols & 31))
        return set_error(FLH_ERR_UNSUPPORTED, "32-block int8 dot: cols must be a multiple of 32, <= 16384");
    if (a0.rows == 0 || a0.nx == 0) return FLH_OK;
    for (uint32_t p0 = 0; p0 < a0.nx; p0 += 4) {
        DotArgs a = a0;
        a.nx = a0.nx - p0 < 4 ? a0.nx - p0 : 4;
        a.x = a0.x + (size_t)p0 * a0.xstride;
        a.y = a0.y + (size_t)p0 * a0.ystride;
        int rc;
        if (nb <= 256) rc = a.nx == 1 ? launch_q8<FMT, 1, 1>(a, s) : a.nx == 2 ? launch_q8<FMT, 2, 1>(a, s) : launch_q8<FMT, 4, 1>(a, s);
        else           rc = a.nx == 1 ? launch_q8<FMT, 1, 2>(a, s) : a.nx == 2 ? launch_q8<FMT, 2, 2>(a, s) : launch_q8<FMT, 4, 2>(a, s);
        if (rc) return rc;
    }
    return FLH_OK;
}

int launch_dot_i8_q8_0(const DotArgs & a, hipStream_t s) { return launch_i8_b32<FMT_Q8_0>(a, s); }
int launch_dot_i8_q5_0(const DotArgs & a, hipStream_t s) { return launch_i8_b32<FMT_Q5_0>(a, s); }
int launch_dot_i8_iq(int fmt, const DotArgs & a, hipStream_t s) {
    if (a.cols & 255) return set_error(FLH_ERR_UNSUPPORTED, "IQ int8 dot: cols must be a multiple of 256");
    if (fmt == FMT_IQ2_XXS) return launch_i8_b32<FMT_IQ2_XXS>(a, s);
    if (fmt == FMT_IQ3_XXS) return launch_i8_b32<FMT_IQ3_XXS>(a, s);
    return set_error(FLH_ERR_UNSUPPORTED, "IQ int8 dot: IQ2_XXS / IQ3_XXS only");
}

}  // namespace flh
