// flh_f32.hip -- fp32-activation STREAM_DOT modes and the small decode ops.
//
//  * canonical (fast = 0): one thread per (row, column) runs the reference's
//    single-accumulator ascending-element chain (fl_dot_row_any,
//    src/runtime/quants.h:132-230,625-642), so it is bitwise equal to
//    run_serial.  Inherently serial per row; it is the reference's
//    correctness mode, not a throughput path.
//  * fast fp32 (fast = 1, format not routed to an int8 path): the
//    reference's fixed 16-lane order (src/runtime/kernels.h:11-19):
//    dot_row_fast / dot_row_fast_q8_0 / dot_row_fast_dequant, bitwise: the
//    256-element chunk formats (Q4_K, Q6_K -- the reference GPU masks' Q6_K
//    route --, Q5_0, IQ2_XXS, IQ3_XXS) on one wave per row (k_dot_fastk),
//    F32 (e.g. an MoE router) and Q8_0 on 16 lanes per row (k_dot_f32row).
//  * ROUTER_SEL / SILU_MUL / WMERGE / MERGE: the reference's single-thread
//    canonical ops (src/runtime/decode_params.h:234-295,
//    runtime_internal.h:274-281), one thread per token / element.  expf is
//    the device libm (the reference runs glibc's), so these match to within
//    float rounding of expf, not bitwise.
#include "flh_common.h"
#include "flh_internal.h"
#include "flh_status.h"
#include "flh_kstream.h"

#include <algorithm>
#include <utility>

namespace flh {

__device__ __forceinline__ uint32_t ld16u(const uint8_t * p) { return p[0] | (p[1] << 8); }

// Q5_0 value of element j (0..31) of a block: 4 bits from qs, the 5th from
// bit j of qh, minus 16 (src/runtime/kernels.h:169-180)
__device__ __forceinline__ int q5v(const uint8_t * b, uint32_t qh, int j) {
    if (j < 16) return (int)((b[6 + j] & 0x0F) | (((qh >> j) << 4) & 0x10)) - 16;
    return (int)((b[6 + j - 16] >> 4) | ((qh >> (j - 4)) & 0x10)) - 16;
}
__device__ __forceinline__ uint32_t q5qh(const uint8_t * b) {
    return b[2] | (b[3] << 8) | (b[4] << 16) | ((uint32_t)b[5] << 24);
}

__device__ float canon_dot(int fmt, const uint8_t * row, const float * x, uint32_t cols) {
    float acc = 0.f;
    if (fmt == FMT_F32) {
        const float * r = (const float *)row;
        for (uint32_t c = 0; c < cols; ++c) acc += r[c] * x[c];
    } else if (fmt == FMT_Q8_0) {
        for (uint32_t b = 0; b < cols / 32; ++b) {
            const uint8_t * B = row + (size_t)b * 34;
            const float d = h2f(ld16u(B));
            for (int i = 0; i < 32; ++i) acc += d * (float)(int8_t)B[2 + i] * x[b * 32 + i];
        }
    } else if (fmt == FMT_Q5_0) {       // fl_dot_row_q5_0, src/runtime/quants.h:144-162
        for (uint32_t b = 0; b < cols / 32; ++b) {
            const uint8_t * B = row + (size_t)b * 22;
            const float d = h2f(ld16u(B));
            const uint32_t qh = q5qh(B);
            for (int j = 0; j < 32; ++j) acc += d * (float)q5v(B, qh, j) * x[b * 32 + j];
        }
    } else if (fmt == FMT_IQ2_XXS || fmt == FMT_IQ3_XXS) {
        // fl_dot_row_iq2_xxs / fl_dot_row_iq3_xxs (src/runtime/quants.h:237-290):
        // IQ2 ascending; IQ3 element 8l+j then 8l+j+4 for j = 0..3
        const uint32_t bb = iq_block_bytes(fmt);
        for (uint32_t sb = 0; sb < cols / 256; ++sb) {
            const uint8_t * B = row + (size_t)sb * bb;
            const float * xb = x + sb * 256;
            const float d = h2f(ld16u(B));
            for (int ib = 0; ib < 8; ++ib) {
                const uint32_t w1 = iq_w1(fmt, B, ib);
                const float db = iq_db(fmt, d, w1);
                for (int l = 0; l < 4; ++l) {
                    if (fmt == FMT_IQ2_XXS) {
                        for (int j = 0; j < 8; ++j) {
                            const int e = 8 * l + j;
                            acc += db * (float)iq_val(fmt, B, ib, w1, e) * xb[32 * ib + e];
                        }
                    } else {
                        for (int j = 0; j < 4; ++j) {
                            const int e1 = 8 * l + j, e2 = e1 + 4;
                            acc += db * (float)iq_val(fmt, B, ib, w1, e1) * xb[32 * ib + e1];
                            acc += db * (float)iq_val(fmt, B, ib, w1, e2) * xb[32 * ib + e2];
                        }
                    }
                }
            }
        }
    } else if (fmt == FMT_Q4_K) {
        for (uint32_t sb = 0; sb < cols / 256; ++sb) {
            const uint8_t * B = row + (size_t)sb * 144;
            const float d = h2f(ld16u(B)), dmin = h2f(ld16u(B + 2));
            const uint8_t * s = B + 4;
            for (int c = 0; c < 4; ++c) {
                uint32_t sc[2], mn[2];
                for (int t = 0; t < 2; ++t) {
                    const int g = 2 * c + t;
                    if (g < 4) { sc[t] = s[g] & 63; mn[t] = s[g + 4] & 63; }
                    else { sc[t] = (s[g + 4] & 0xF) | ((s[g - 4] >> 6) << 4);
                           mn[t] = (s[g + 4] >> 4) | ((s[g] >> 6) << 4); }
                }
                const float d1 = d * (float)sc[0], m1 = dmin * (float)mn[0];
                const float d2 = d * (float)sc[1], m2 = dmin * (float)mn[1];
                const uint8_t * q = B + 16 + 32 * c;
                const float * xb = x + sb * 256 + 64 * c;
                for (int l = 0; l < 32; ++l) acc += (d1 * (float)(q[l] & 0xF) - m1) * xb[l];
                for (int l = 0; l < 32; ++l) acc += (d2 * (float)(q[l] >> 4) - m2) * xb[32 + l];
            }
        }
    } else {
        for (uint32_t sb = 0; sb < cols / 256; ++sb) {
            const uint8_t * B = row + (size_t)sb * 210;
            const float d = h2f(ld16u(B + 208));
            const int8_t * sc = (const int8_t *)(B + 192);
            for (int h = 0; h < 2; ++h)
                for (int g = 0; g < 4; ++g)
                    for (int l = 0; l < 32; ++l) {
                        const uint8_t lb = B[64 * h + l + 32 * (g & 1)];
                        const int q6 = ((g < 2) ? (lb & 0xF) : (lb >> 4)) |
                                       (((B[128 + 32 * h + l] >> (2 * g)) & 3) << 4);
                        acc += d * (float)sc[8 * h + 2 * g + l / 16] * (float)(q6 - 32)
                             * x[sb * 256 + 128 * h + 32 * g + l];
                    }
        }
    }
    return acc;
}

// K formats on the q8_1 int8 path (i8 mask bit set, i8k bit clear):
// fl_dot_i8_q4_K / fl_dot_i8_q6_K (src/runtime/quants.h:468-526), exact
// integer group sums, two (Q4_K) or per-16 (Q6_K) fmaf terms per 32-element
// block into acc[. & 3], fold (a0 + a1) + (a2 + a3).  The reference's default
// masks never route here; one thread per (row, column), bitwise.
__device__ float q81k_dot(int fmt, const uint8_t * row, const uint8_t * xq, uint32_t cols) {
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t sb = 0; sb < cols / 256; ++sb) {
        if (fmt == FMT_Q4_K) {
            const uint8_t * W = row + (size_t)sb * 144;
            const float d = h2f(ld16u(W)), dmin = h2f(ld16u(W + 2));
            const uint8_t * s = W + 4;
            for (int g = 0; g < 8; ++g) {
                uint32_t sc, mn;
                if (g < 4) { sc = s[g] & 63; mn = s[g + 4] & 63; }
                else { sc = (s[g + 4] & 0xF) | ((s[g - 4] >> 6) << 4); mn = (s[g + 4] >> 4) | ((s[g] >> 6) << 4); }
                const uint8_t * q = W + 16 + (g / 2) * 32;
                const uint8_t * X = xq + (size_t)(sb * 8 + g) * 36;
                int idot = 0, isum = 0;
                for (int i = 0; i < 32; ++i) {
                    const int w4 = (g & 1) ? (q[i] >> 4) : (q[i] & 0xF);
                    idot += w4 * (int8_t)X[4 + i];
                    isum += (int8_t)X[4 + i];
                }
                const float dx = h2f(ld16u(X));
                a[g & 3] = fmaf(d * (float)sc * dx, (float)idot, a[g & 3]);
                a[g & 3] = fmaf(-(dmin * (float)mn) * dx, (float)isum, a[g & 3]);
            }
        } else {
            const uint8_t * W = row + (size_t)sb * 210;
            const float d = h2f(ld16u(W + 208));
            const int8_t * sc = (const int8_t *)(W + 192);
            for (int h = 0; h < 2; ++h)
                for (int g = 0; g < 4; ++g) {
                    const uint8_t * X = xq + (size_t)(sb * 8 + h * 4 + g) * 36;
                    const float dx = h2f(ld16u(X));
                    for (int k = 0; k < 2; ++k) {
                        int idot = 0, isum = 0;
                        for (int i = 0; i < 16; ++i) {
                            const int e = 16 * k + i;
                            const uint8_t lb = W[64 * h + e + 32 * (g & 1)];
                            const int q6 = ((g < 2) ? (lb & 0xF) : (lb >> 4)) |
                                           (((W[128 + 32 * h + e] >> (2 * g)) & 3) << 4);
                            idot += q6 * (int8_t)X[4 + e];
                            isum += (int8_t)X[4 + e];
                        }
                        const int t = (int)sc[8 * h + 2 * g + k] * (idot - 32 * isum);
                        const int ti = 8 * h + 2 * g + k;
                        a[ti & 3] = fmaf(d * dx, (float)t, a[ti & 3]);
                    }
                }
        }
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

__global__ void k_dot_q81k(int fmt, DotArgs a) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (uint64_t)a.rows * a.nx) return;
    const uint32_t r = (uint32_t)(t % a.rows), p = (uint32_t)(t / a.rows);
    const uint8_t * w = a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0);
    const uint64_t rb = (uint64_t)(a.cols / 256) * (fmt == FMT_Q4_K ? 144 : 210);
    const uint8_t * xq = (const uint8_t *)(a.x + (size_t)p * a.xstride) + xq_off(a.cols);
    const float v = q81k_dot(fmt, w + r * rb, xq, a.cols);
    float * y = a.y + (size_t)p * a.ystride + r;
    *y = *y + v;
}

int launch_dot_i8_k(int fmt, const DotArgs & a, hipStream_t s) {
    if (fmt != FMT_Q4_K && fmt != FMT_Q6_K) return set_error(FLH_ERR_UNSUPPORTED, "q8_1 K-format dot: Q4_K / Q6_K only");
    const uint64_t n = (uint64_t)a.rows * a.nx;
    if (n == 0) return FLH_OK;
    hipLaunchKernelGGL(k_dot_q81k, dim3((uint32_t)((n + 63) / 64)), dim3(64), 0, s, fmt, a);
    return hip_check(hipGetLastError(), "k_dot_q81k launch");
}

// Fast fp32 order of the K formats (dot_row_fast_dequant: dequant_chunk of
// each 256-element chunk, dot_row_fast's 16 partial sums and tree, chunk
// sums added in order; src/runtime/kernels.h:59-104,162-254) on one wave per
// row and all of its columns: a chunk on 16 lanes, lane j owning elements
// j + 16 k (k = 0..15, so that its partial sum is the reference's L[j]),
// four chunks per pass; the value of each element is computed as
// dequant_chunk does (Q4_K: (d sc) q - (dmin m); Q6_K: (d sc) (q - 32); Q5_0:
// d (q - 16); IQ: db (+-v)), and every product and sum rounds on its own.
//
// Memory plan: the four superblocks of a pass arrive as one 16-byte load per
// lane (the aligned 16-byte segments that cover them; a segment holding one
// byte of the row lies in that byte's page), issued two passes ahead into two
// registers used in turn (a register copy would wait for its load), and go
// through a 1 KiB wave-private LDS buffer from which each lane picks its
// bytes.  The per-subblock factors d sc (and dmin m) are computed once per
// chunk, by lane k of the chunk's 16, and reach the other 15 lanes by DPP
// row broadcasts.  The workgroup's four waves run R consecutive rows each,
// tile by tile: a tile is T superblocks of the activations, staged in LDS by
// the whole workgroup (chunks 272 floats apart, so the four chunks of a pass
// read disjoint bank halves); a row's running sum waits in lane rr of a
// register between its tiles, and y is read and written once, at the end.
__host__ __device__ constexpr uint32_t fk_chunk_bytes(int fmt) {
    return fmt == FMT_Q4_K ? 144u : fmt == FMT_Q6_K ? 210u : fmt == FMT_Q5_0 ? 176u
         : fmt == FMT_IQ2_XXS ? 66u : 98u;
}
__host__ __device__ constexpr uint32_t fk_grid_bytes(int fmt) {
    return fmt == FMT_IQ2_XXS ? 2048u : fmt == FMT_IQ3_XXS ? 1024u : 0u;
}
constexpr uint32_t FK_WBUF = 1024;      // staging bytes per wave (<= 64 segments)
constexpr uint32_t FK_XPAD = 272;       // floats per staged activation chunk
constexpr uint32_t FK_XT_BYTES = 32768; // activation tile budget, bytes

template <int K> __device__ __forceinline__ float row_bcast(float v) {
    // lane K of each 16-lane row, to the whole row (DPP row_newbcast)
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + K, 0xF, 0xF, false));
}
// four bytes b0 | b1 << 8 | b2 << 16 | b3 << 24, built as two 16-bit pairs
// (b0, b2) and (b1, b3): two v_perm_b32 and one shift-or
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack4(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
    u16x2 e, o;
    e.x = (uint16_t)b0; e.y = (uint16_t)b2;
    o.x = (uint16_t)b1; o.y = (uint16_t)b3;
    return __builtin_bit_cast(uint32_t, e) | (__builtin_bit_cast(uint32_t, o) << 8);
}
template <typename F, int... K>
__device__ __forceinline__ void static_for(F && f, std::integer_sequence<int, K...>) {
    (f(std::integral_constant<int, K>()), ...);
}

template <int FMT, int NXT>
__global__ __launch_bounds__(256) void k_dot_fastk(DotArgs a, uint32_t R, uint32_t T) {
    // NXT: column slots (1, 2, 4; a.nx <= NXT)
    static_assert(FMT == FMT_Q4_K || FMT == FMT_Q6_K || FMT == FMT_Q5_0 || FMT == FMT_IQ2_XXS ||
                  FMT == FMT_IQ3_XXS, "formats of the 256-element chunk order");
    extern __shared__ __align__(16) uint8_t fk_smem[];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform, in an SGPR
    const uint32_t j = lane & 15, cq = lane >> 4;
    constexpr uint32_t BB = fk_chunk_bytes(FMT);                  // bytes of a 256-element chunk
    constexpr uint32_t GB = fk_grid_bytes(FMT);                   // IQ codebook staged in LDS
    const uint32_t cols = a.cols, nsb = (cols + 255) >> 8, nx = NXT == 1 ? 1 : a.nx;
    // row bytes (Q5_0: the last chunk holds cols % 256 / 32 blocks)
    const uint32_t RB = FMT == FMT_Q5_0 ? (cols / 32) * 22 : nsb * BB;
    constexpr int NP = NXT;                                       // column slots
    uint8_t * gl = fk_smem + 4 * FK_WBUF;                         // codebook (IQ)
    float * xs = reinterpret_cast<float *>(fk_smem + 4 * FK_WBUF + GB);
    uint8_t * wb = fk_smem + wave * FK_WBUF;
    const uint32_t r0 = (blockIdx.x * 4 + wave) * R;
    const uint32_t nr = r0 < a.rows ? min(R, a.rows - r0) : 0;    // rows of this wave (uniform)
    const uint8_t * wr = a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0) + (size_t)r0 * RB;
    const uint32_t ntile = (nsb + T - 1) / T;
    auto tpass = [&](uint32_t t) { return (min(T, nsb - t * T) + 3) >> 2; };
    const uint32_t NI = nr * ((nsb + 3) >> 2);                    // T % 4 == 0: no pass straddles tiles

    // item = pass ps of tile t of row rr; cursor order t, rr, ps
    struct Cur { uint32_t t, rr, ps; };
    auto start = [&](const Cur & c) { return wr + (size_t)c.rr * RB + (c.t * T + 4 * c.ps) * BB; };
    auto len = [&](const Cur & c) { return min(4 * BB, RB - (c.t * T + 4 * c.ps) * BB); };
    auto advance = [&](Cur & c) {
        if (++c.ps == tpass(c.t)) { c.ps = 0; if (++c.rr == nr) { c.rr = 0; ++c.t; } }
    };
    // every lane loads (lanes past the item's segments repeat its last one)
    // and every step fetches (past the wave's last item, that item again),
    // so the loads are unconditional and their counts known to the compiler
    auto fetch = [&](const Cur & c, u32x4a & v) {
        const uintptr_t A = (uintptr_t)start(c), a0 = A & ~(uintptr_t)15;
        const uint32_t nseg = (uint32_t)((A + len(c) - a0 + 15) >> 4);
        v = *reinterpret_cast<const __attribute__((address_space(1))) u32x4a *>(a0 + 16 * min(lane, nseg - 1));
    };
    Cur fc = {0, 0, 0}, cc = {0, 0, 0};                            // fetch / compute cursors
    uint32_t nf = 0;                                              // items fetched
    auto fetch_next = [&](u32x4a & v) { fetch(fc, v); if (++nf < NI) advance(fc); };
    u32x4a vA = {0, 0, 0, 0}, vB = vA;
    if (NI > 0) { fetch_next(vA); fetch_next(vB); }

    // activation tile t, staged by the whole workgroup: every wave stages
    // tiles 0 .. ntile - 1 in order (at its first item of the tile, or after
    // its items when it has fewer tiles' worth), so the barriers pair up
    uint32_t nt = 0;
    auto stage = [&]() {
        const uint32_t t = nt++;
        if (t > 0) lds_barrier();                                 // all reads of tile t - 1 done
        if constexpr (GB > 0) {
            if (t == 0) {
                const uint32_t * g = FMT == FMT_IQ2_XXS ? reinterpret_cast<const uint32_t *>(k_iq2_grid)
                                                        : reinterpret_cast<const uint32_t *>(k_iq3_grid);
                for (uint32_t i = threadIdx.x; i < GB / 4; i += 256) reinterpret_cast<uint32_t *>(gl)[i] = g[i];
            }
        }
        const uint32_t tc = min(T * 256, cols - t * T * 256);     // elements of the tile
        for (uint32_t p = 0; p < nx; ++p) {
            const float * xp = a.x + (size_t)p * a.xstride + (size_t)t * T * 256;
            for (uint32_t e0 = threadIdx.x; e0 < tc; e0 += 8 * 256) {   // 8 loads in flight
                float r[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) r[u] = e0 + 256 * u < tc ? xp[e0 + 256 * u] : 0.f;
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (e0 + 256 * u < tc) xs[(p * T + (e0 >> 8) + u) * FK_XPAD + (e0 & 255)] = r[u];
            }
        }
        lds_barrier();
    };

    float acc[NP], accv[NP];                                      // running sum (uniform) / per-row sums in lane rr
#pragma unroll
    for (int p = 0; p < NP; ++p) { acc[p] = 0.f; accv[p] = 0.f; }

    auto step = [&](u32x4a & seg) {
        if (cc.rr == 0 && cc.ps == 0 && cc.t == nt) stage();
        const uintptr_t A = (uintptr_t)start(cc);
        const uint32_t sh = (uint32_t)(A & 15);
        *reinterpret_cast<u32x4a *>(wb + 16 * lane) = seg;
        fetch_next(seg);
        __builtin_amdgcn_wave_barrier();
        if (cc.ps == 0) {                                         // a row's segment starts
#pragma unroll
            for (int p = 0; p < NP; ++p)
                if ((uint32_t)p < nx) acc[p] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(accv[p]), cc.rr));
        }
        const uint32_t cl = 4 * cc.ps + cq;                       // chunk within the tile
        const uint32_t c0 = cc.t * T + 4 * cc.ps;
        const bool act = c0 + cq < nsb;
        const uint8_t * b = wb + sh + cq * BB;
        float v[16];
        // elements of the lane's chain in this chunk (Q5_0: the row's last
        // chunk may hold fewer than 256)
        const uint32_t nk = FMT == FMT_Q5_0 ? (act ? min(16u, (cols - 256 * (c0 + cq)) / 16) : 0u) : 16u;
        if constexpr (FMT == FMT_Q5_0) {
            // block k >> 1 of the chunk, element 16 (k & 1) + j: nibble (k & 1 ?
            // high : low) of qs byte j, bit 16 (k & 1) + j of qh, minus 16
            // (dequant_chunk's d * q5); lane g < 8 reads block g's d and qh
            const uint32_t g = j & 7;
            const uint8_t * bg = b + 22 * g;
            const float dg = h2f(*reinterpret_cast<const uint16_t *>(bg));
            const uint32_t qhg = *reinterpret_cast<const uint16_t *>(bg + 2) |
                                 ((uint32_t)*reinterpret_cast<const uint16_t *>(bg + 4) << 16);
            uint32_t qs[8];
#pragma unroll
            for (int m = 0; m < 8; ++m) qs[m] = b[22 * m + 6 + j];
            static_for([&](auto kc) {
                constexpr int k = decltype(kc)::value;
                const uint32_t qh = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)qhg, 0x150 + (k >> 1), 0xF, 0xF, false);
                const uint32_t nib = (k & 1) ? (qs[k >> 1] >> 4) : (qs[k >> 1] & 0xF);
                const int q = (int)(nib | (((qh >> (16 * (k & 1) + j)) & 1u) << 4)) - 16;
                v[k] = row_bcast<(k >> 1)>(dg) * (float)q;
            }, std::make_integer_sequence<int, 16>());
        } else if constexpr (FMT == FMT_IQ2_XXS || FMT == FMT_IQ3_XXS) {
            // group ib = k >> 1, element 16 (k & 1) + j: run l = 2 (k & 1) +
            // (j >> 3), magnitude byte j & 7 (IQ2: of the 8-byte codebook entry
            // of index byte l) or j & 3 (IQ3: of the 4-byte entry of index byte
            // 2 l + ((j >> 2) & 1)), sign bit 16 (k & 1) + j of the group's four
            // parity-widened 7-bit fields; value db * (+-magnitude).  Lane g < 8
            // makes group g's db and sign bytes
            const uint32_t g = j & 7;
            const float d = h2f(*reinterpret_cast<const uint16_t *>(b));
            const uint8_t * wp = FMT == FMT_IQ2_XXS ? b + 2 + 8 * g + 4 : b + 66 + 4 * g;
            const uint32_t w1 = *reinterpret_cast<const uint16_t *>(wp) |
                                ((uint32_t)*reinterpret_cast<const uint16_t *>(wp + 2) << 16);
            const float dbg = FMT == FMT_IQ2_XXS ? (d * (0.5f + (float)(w1 >> 28))) * 0.25f
                                                 : (d * (0.5f + (float)(w1 >> 28))) * 0.5f;
            const uint32_t sgg = iq_sign8(w1) | (iq_sign8(w1 >> 7) << 8) | (iq_sign8(w1 >> 14) << 16) |
                                 (iq_sign8(w1 >> 21) << 24);
            static_for([&](auto kc) {
                constexpr int k = decltype(kc)::value;
                constexpr int ib = k >> 1;
                uint32_t mag;
                if constexpr (FMT == FMT_IQ2_XXS) mag = gl[8 * b[2 + 8 * ib + 2 * (k & 1) + (j >> 3)] + (j & 7)];
                else mag = gl[4 * b[2 + 8 * ib + 4 * (k & 1) + (j >> 2)] + (j & 3)];
                const uint32_t sg = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)sgg, 0x150 + ib, 0xF, 0xF, false);
                const float m = (float)mag;
                v[k] = row_bcast<ib>(dbg) * (((sg >> (16 * (k & 1) + j)) & 1u) ? -m : m);
            }, std::make_integer_sequence<int, 16>());
        } else if constexpr (FMT == FMT_Q6_K) {
            // element k = 8 h + 2 g + o of the lane: 4 low bits from the low
            // (g < 2) or high nibble of ql byte 64 h + 16 (o + 2 (g & 1)) + j,
            // 2 high bits from bits 2 g of qh byte 128 + 32 h + 16 o + j.  Per
            // half, the four ql bytes are packed into QL (byte m = o + 2 (g & 1))
            // and the two qh bytes into Y so that byte m of Y's bits 0-1 (4-5)
            // are the high bits of the low (high) nibble's element.  Each byte
            // of Q is then (q6 ^ 0x20) << 2, i.e. 4 (q6 - 32) as a signed byte,
            // and the factor is d sc / 4: (d sc / 4) (4 (q6 - 32)) is the same
            // product as (d sc) (q6 - 32), rounded once (d sc / 4 is exact:
            // |d sc| >= 2^-24 or 0).
            const float d = h2f(*reinterpret_cast<const uint16_t *>(b + 208));
            const float dd4 = (d * (float)(int8_t)b[192 + j]) * 0.25f;
            uint32_t Q[4];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t QL = pack4(b[64 * h + j], b[64 * h + 16 + j], b[64 * h + 32 + j], b[64 * h + 48 + j]);
                const uint32_t QHP = b[128 + 32 * h + j] | (b[128 + 32 * h + 16 + j] << 8);
                // bits 0-1 and 4-5 of each byte, bit 1 / 5 flipped (q6 ^ 0x20)
                const uint32_t Y = ((QHP | (QHP << 14)) ^ 0x22222222u) & 0x33333333u;
                Q[2 * h] = ((QL << 2) & 0x3C3C3C3Cu) | ((Y << 6) & 0xC0C0C0C0u);
                Q[2 * h + 1] = ((QL >> 2) & 0x3C3C3C3Cu) | ((Y << 2) & 0xC0C0C0C0u);
            }
            static_for([&](auto kc) {
                constexpr int k = decltype(kc)::value;
                constexpr int h = k >> 3, g = (k >> 1) & 3, o = k & 1, m = o + 2 * (g & 1);
                const int q = (int8_t)(Q[2 * h + (g >> 1)] >> (8 * m));
                v[k] = row_bcast<k>(dd4) * (float)q;
            }, std::make_integer_sequence<int, 16>());
        } else {
            // element k: nibble (k & 2 ? high : low) of qs byte
            // 16 + 32 (k >> 2) + 16 (k & 1) + j, subblock k >> 1
            const float d = h2f(*reinterpret_cast<const uint16_t *>(b)), dmin = h2f(*reinterpret_cast<const uint16_t *>(b + 2));
            const uint8_t * sp = b + 4;
            const uint32_t g = j & 7;
            uint32_t sc, mn;
            if (g < 4) { sc = sp[g] & 63; mn = sp[g + 4] & 63; }
            else { sc = (sp[g + 4] & 0xF) | ((sp[g - 4] >> 6) << 4); mn = (sp[g + 4] >> 4) | ((sp[g] >> 6) << 4); }
            const float ddg = d * (float)sc, mmg = dmin * (float)mn;
            uint32_t N[4];                    // low / high nibbles of bytes 4 t .. 4 t + 3 of the 8
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint32_t QS = pack4(b[16 + 64 * t + j], b[32 + 64 * t + j], b[48 + 64 * t + j], b[64 + 64 * t + j]);
                N[2 * t] = QS & 0x0F0F0F0Fu;
                N[2 * t + 1] = (QS >> 4) & 0x0F0F0F0Fu;
                // keep the masks out of sight so each nibble converts in one
                // v_cvt_f32_ubyteN (folded, they become a shift, a mask and a convert)
                asm volatile("" : "+v"(N[2 * t]), "+v"(N[2 * t + 1]));
            }
            static_for([&](auto kc) {
                constexpr int k = decltype(kc)::value;
                constexpr int m = 2 * (k >> 2) + (k & 1);             // byte of the 8
                const uint32_t nib = (N[2 * (m >> 2) + ((k >> 1) & 1)] >> (8 * (m & 3))) & 0xFF;
                v[k] = row_bcast<(k >> 1)>(ddg) * (float)nib - row_bcast<(k >> 1)>(mmg);
            }, std::make_integer_sequence<int, 16>());
        }
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            if ((uint32_t)p >= nx) continue;                      // uniform
            const float * x = xs + (p * T + (act ? cl : 0)) * FK_XPAD + j;
            float L = 0.f;
            if constexpr (FMT == FMT_Q5_0) {
#pragma unroll
                for (int k = 0; k < 16; ++k) L = (uint32_t)k < nk ? L + v[k] * x[16 * k] : L;
            } else {
#pragma unroll
                for (int k = 0; k < 16; ++k) L = L + v[k] * x[16 * k];
            }
            // tree16 on the 16 lanes of the chunk: lane 0 ends with
            // ((L0 + L4) + (L8 + L12)) + ... as dot_row_fast's
            // (lanes past the row's end read 0: bound_ctrl, so the shift
            // folds into the add as its DPP operand; lane 0 reads none of them)
            const float u = L + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(L), 0x104, 0xF, 0xF, true));
            const float t = u + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(u), 0x108, 0xF, 0xF, true));
            const float h2 = t + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0x101, 0xF, 0xF, true));
            const float head = h2 + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(h2), 0x102, 0xF, 0xF, true));
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (c0 + q < nsb) acc[p] = acc[p] + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(head), 16 * q));
        }
        const Cur done = cc;
        advance(cc);
        if (cc.ps == 0) {                                         // the row's segment ends
#pragma unroll
            for (int p = 0; p < NP; ++p)
                if ((uint32_t)p < nx) accv[p] = lane == done.rr ? acc[p] : accv[p];
        }
    };

    uint32_t it = 0;
    for (; it + 1 < NI; it += 2) { step(vA); step(vB); }          // two registers in turn
    if (it < NI) step(vA);
    while (nt < ntile) stage();
    if (lane < nr) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            if ((uint32_t)p >= nx) continue;
            float * y = a.y + (size_t)p * a.ystride + r0 + lane;
            *y = *y + accv[p];
        }
    }
}

// Fast fp32 order of F32 and Q8_0 weights (dot_row_fast and
// dot_row_fast_q8_0, src/runtime/kernels.h:11-19,58-130: L[j] over the
// elements k < n16 with k % 16 == j in ascending k -- for Q8_0 the product
// (d q) x of each element -- the 16-lane tree, then for F32 the tail k >= n16
// in order, y += head + tail): the route of every F32 matrix (e.g. an MoE
// router) under every mask, and of Q8_0 without its int8 bit.  16 lanes per
// row, lane j running L[j]; a wave holds 4 rows, a workgroup 16.  A block is
// 256 columns (16 elements per lane), loaded 2-4 blocks ahead into register
// sets used in turn (F32: 16 dword loads per lane; Q8_0: 16 byte loads and the
// 8 block scales); the activations are staged in LDS by the workgroup in
// tiles of up to 32 KB (every row of a wave reads the same address: a
// broadcast).  Elements past n16 are masked out of the chains (their loads
// read a valid address).
constexpr uint32_t F32R_XT_BYTES = 32768;

template <int FMT, int NXT, int D>
__global__ __launch_bounds__(256) void k_dot_f32row(DotArgs a, uint32_t T) {
    // NXT: column slots (1, 2, 4; a.nx <= NXT); D: blocks in flight
    static_assert(FMT == FMT_F32 || FMT == FMT_Q8_0, "F32 / Q8_0");
    extern __shared__ __align__(16) uint8_t f32r_smem[];
    float * xs = reinterpret_cast<float *>(f32r_smem);
    const uint32_t lane = threadIdx.x & 63, j = lane & 15;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr int NP = NXT;
    const uint32_t nx = NXT == 1 ? 1 : a.nx, cols = a.cols, n16 = cols & ~15u;
    const uint32_t RB = FMT == FMT_F32 ? cols * 4 : (cols / 32) * 34;          // row bytes
    const uint32_t r = blockIdx.x * 16 + wave * 4 + (lane >> 4);
    const uint32_t rw = min(blockIdx.x * 16 + wave * 4, a.rows - 1);   // the wave's first row (uniform)
    const uint8_t * w0 = a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0) + (size_t)rw * RB;
    const uint32_t roff = (min(r, a.rows - 1) - rw) * RB;        // < 4 rows: 32 bits
    const auto * wg = (const __attribute__((address_space(1))) uint8_t *)w0;
    const uint32_t nblk = (n16 + 255) / 256;                      // blocks of 256 columns
    using u32x16 = uint32_t __attribute__((ext_vector_type(16)));
    using u32x8 = uint32_t __attribute__((ext_vector_type(8)));
    struct Blk { u32x16 q; u32x8 d; };                            // F32: q holds the values' bits
    auto fetch = [&](uint32_t kb, Blk & v) __attribute__((always_inline)) {   // block min(kb, nblk - 1), clamped reads
        const uint32_t c0 = min(kb, nblk - 1) * 256 + j;
        if constexpr (FMT == FMT_F32) {
#pragma unroll
            for (int e = 0; e < 16; ++e)
                v.q[e] = *(const __attribute__((address_space(1))) uint32_t *)(wg + roff + 4 * min(c0 + 16 * e, cols - 1));
        } else {
            const uint32_t b0 = min(kb, nblk - 1) * 8, nb = cols / 32;
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const uint32_t ob = roff + 34 * min(b0 + m, nb - 1);
                v.d[m] = *(const __attribute__((address_space(1))) uint16_t *)(wg + ob);
                v.q[2 * m] = wg[ob + 2 + j];
                v.q[2 * m + 1] = wg[ob + 18 + j];
            }
        }
    };
    float L[NP], yv[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        L[p] = 0.f;
        // the old y, requested before any weight (only this lane writes it)
        yv[p] = (uint32_t)p < nx && r < a.rows ? a.y[(size_t)p * a.ystride + r] : 0.f;
    }
    uint32_t nt = 0;                                              // tiles staged
    auto stage = [&](uint32_t t) __attribute__((always_inline)) {
        if (t > 0) lds_barrier();
        const uint32_t c0 = t * T, tc = min(T, n16 - c0);
        for (uint32_t p = 0; p < nx; ++p) {
            const float * xp = a.x + (size_t)p * a.xstride + c0;
            for (uint32_t e0 = threadIdx.x; e0 < tc; e0 += 8 * 256) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = e0 + 256 * u < tc ? xp[e0 + 256 * u] : 0.f;
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (e0 + 256 * u < tc) xs[p * T + e0 + 256 * u] = v[u];
            }
        }
        lds_barrier();
    };
    auto step = [&](uint32_t kb, Blk & v) __attribute__((always_inline)) {
        if (kb * 256 == nt * T) stage(nt++);
        float w[16];
        if constexpr (FMT == FMT_F32) {
#pragma unroll
            for (int e = 0; e < 16; ++e) w[e] = __uint_as_float(v.q[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) w[e] = h2f(v.d[e >> 1]) * (float)(int8_t)v.q[e];   // d q
        }
        fetch(kb + D, v);
        const uint32_t c = kb * 256 - (nt - 1) * T;               // column of the block within its tile
        const bool full = kb * 256 + 256 <= n16;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            if ((uint32_t)p >= nx) continue;
            const float * x = xs + p * T + c + j;
            float l = L[p];
            if (full) {
#pragma unroll
                for (int e = 0; e < 16; ++e) l = l + w[e] * x[16 * e];
            } else {
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    if (kb * 256 + 16 * e < n16) l = l + w[e] * x[16 * e];   // uniform
            }
            L[p] = l;
        }
    };
    Blk v[D];                                                     // block kb in v[kb % D]
    if (nblk > 0) static_for([&](auto ic) { fetch(decltype(ic)::value, v[decltype(ic)::value]); },
                             std::make_integer_sequence<int, D>());
    uint32_t kb = 0;
    for (; kb + D <= nblk; kb += D)
        static_for([&](auto ic) { step(kb + decltype(ic)::value, v[decltype(ic)::value]); },
                   std::make_integer_sequence<int, D>());
    static_for([&](auto ic) { if (kb + decltype(ic)::value < nblk) step(kb + decltype(ic)::value, v[decltype(ic)::value]); },
               std::make_integer_sequence<int, D>());
    if (r >= a.rows) return;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        if ((uint32_t)p >= nx) continue;
        const float Lp = L[p];
        const float u = Lp + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(Lp), 0x104, 0xF, 0xF, true));
        const float t = u + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(u), 0x108, 0xF, 0xF, true));
        const float h2 = t + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0x101, 0xF, 0xF, true));
        const float head = h2 + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(h2), 0x102, 0xF, 0xF, true));
        if (j == 0) {
            float tail = 0.f;
            if constexpr (FMT == FMT_F32) {                       // Q8_0: cols % 32 == 0, no tail
                const float * wr = reinterpret_cast<const float *>(w0 + roff);
                const float * x = a.x + (size_t)p * a.xstride;
                for (uint32_t k = n16; k < cols; ++k) tail = tail + wr[k] * x[k];
            }
            a.y[(size_t)p * a.ystride + r] = yv[p] + (FMT == FMT_F32 ? head + tail : head);
        }
    }
}

__global__ void k_dot_canon(int fmt, DotArgs a) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (uint64_t)a.rows * a.nx) return;
    const uint32_t r = (uint32_t)(t % a.rows), p = (uint32_t)(t / a.rows);
    const uint8_t * w = a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0);
    const uint64_t rb = fmt == FMT_F32 ? (uint64_t)a.cols * 4
                      : fmt == FMT_Q8_0 ? (uint64_t)(a.cols / 32) * 34
                      : fmt == FMT_Q5_0 ? (uint64_t)(a.cols / 32) * 22
                      : (uint64_t)(a.cols / 256) * (fmt == FMT_Q4_K ? 144 : fmt == FMT_Q6_K ? 210
                                                   : iq_block_bytes(fmt));
    const float * x = a.x + (size_t)p * a.xstride;
    const float v = canon_dot(fmt, w + r * rb, x, a.cols);
    float * y = a.y + (size_t)p * a.ystride + r;
    *y = *y + v;
}

static int launch_f32(bool fast, int fmt, const DotArgs & a, hipStream_t s) {
    if (fmt < FMT_F32 || fmt > FMT_IQ3_XXS)
        return set_error(FLH_ERR_UNSUPPORTED, "fp32 dot: format not supported");
    const uint64_t n = (uint64_t)a.rows * a.nx;
    if (n == 0) return FLH_OK;
    const bool chunked = fmt == FMT_Q4_K || fmt == FMT_Q6_K || fmt == FMT_Q5_0 || fmt == FMT_IQ2_XXS ||
                         fmt == FMT_IQ3_XXS;
    if (fast && (chunked || fmt == FMT_F32 || fmt == FMT_Q8_0) && a.nx > 4 && a.nx <= 16) {
        // more than 4 columns: groups of 4, each its own pass over the weights
        // (per column the 4-column launch costs least: the activation tiles of
        // 8 or 16 columns are short, and every tile drains the prefetch)
        for (uint32_t p0 = 0; p0 < a.nx; p0 += 4) {
            DotArgs g = a;
            g.x = a.x + (size_t)p0 * a.xstride;
            g.y = a.y + (size_t)p0 * a.ystride;
            g.nx = std::min(4u, a.nx - p0);
            if (int rc = launch_f32(true, fmt, g, s)) return rc;
        }
        return FLH_OK;
    }
    if (fast && chunked && a.nx <= 4) {
        // T: chunks per activation tile, a multiple of 4, within the tile
        // budget (4 for 8 or more columns); R: rows per wave
        const uint32_t nsb = (a.cols + 255) / 256;
        uint32_t T = std::max(4u, (uint32_t)(FK_XT_BYTES / (a.nx * FK_XPAD * 4)) & ~3u);
        T = std::min(T, std::max(4u, (nsb + 3) & ~3u));          // >= 4 also for rows of no columns
        uint32_t R = std::min(4u, std::max(1u, a.rows / 16384));
        const size_t smem = 4 * FK_WBUF + fk_grid_bytes(fmt) + (size_t)a.nx * T * FK_XPAD * 4;
        const dim3 gw((uint32_t)((a.rows + 4ull * R - 1) / (4ull * R)));
        const uint32_t slots = a.nx == 1 ? 0 : a.nx == 2 ? 1 : 2;
#define FLH_FK_ROW(F) {(const void *)k_dot_fastk<F, 1>, (const void *)k_dot_fastk<F, 2>, (const void *)k_dot_fastk<F, 4>}
        static const void * const kfk[5][3] = {FLH_FK_ROW(FMT_Q4_K), FLH_FK_ROW(FMT_Q6_K), FLH_FK_ROW(FMT_Q5_0),
                                               FLH_FK_ROW(FMT_IQ2_XXS), FLH_FK_ROW(FMT_IQ3_XXS)};
#undef FLH_FK_ROW
        const int fi = fmt == FMT_Q4_K ? 0 : fmt == FMT_Q6_K ? 1 : fmt == FMT_Q5_0 ? 2 : fmt == FMT_IQ2_XXS ? 3 : 4;
        const void * kern = kfk[fi][slots];
        if (int rc = lds_fits(kern, smem, "k_dot_fastk")) return rc;
        void * args[] = {const_cast<DotArgs *>(&a), &R, &T};
        return hip_check(hipLaunchKernel(kern, gw, dim3(256), args, smem, s), "k_dot_fastk launch");
    }
    if (fast && (fmt == FMT_F32 || fmt == FMT_Q8_0) && a.nx <= 4) {
        // the kernel addresses a wave's 4 rows with 32-bit byte offsets
        if ((uint64_t)a.cols * 4 * 4 >= (1ull << 32))
            return set_error(FLH_ERR_UNSUPPORTED, "fast fp32 dot: F32 / Q8_0 rows longer than 2^28 columns");
        // T: columns per activation tile, a multiple of 256 within the budget
        uint32_t T = std::max(256u, (uint32_t)(F32R_XT_BYTES / (4 * a.nx)) & ~255u);
        T = std::min(T, std::max(256u, ((a.cols & ~15u) + 255) & ~255u));
        const size_t smem = (size_t)a.nx * T * 4;
        const dim3 gw((a.rows + 15) / 16);
        const uint32_t slots = a.nx == 1 ? 0 : a.nx == 2 ? 1 : 2;
        static const void * const kf32[3] = {
            (const void *)k_dot_f32row<FMT_F32, 1, 4>, (const void *)k_dot_f32row<FMT_F32, 2, 4>,
            (const void *)k_dot_f32row<FMT_F32, 4, 2>};
        static const void * const kq8[3] = {
            (const void *)k_dot_f32row<FMT_Q8_0, 1, 4>, (const void *)k_dot_f32row<FMT_Q8_0, 2, 4>,
            (const void *)k_dot_f32row<FMT_Q8_0, 4, 2>};
        const void * kern = fmt == FMT_F32 ? kf32[slots] : kq8[slots];
        if (int rc = lds_fits(kern, smem, "k_dot_f32row")) return rc;
        void * args[] = {const_cast<DotArgs *>(&a), &T};
        return hip_check(hipLaunchKernel(kern, gw, dim3(256), args, smem, s), "k_dot_f32row launch");
    }
    if (fast) return set_error(FLH_ERR_UNSUPPORTED, "fast fp32 dot: more than 16 columns");
    hipLaunchKernelGGL(k_dot_canon, dim3((uint32_t)((n + 63) / 64)), dim3(64), 0, s, fmt, a);
    return hip_check(hipGetLastError(), "k_dot_canon launch");
}
int launch_dot_canonical(int fmt, const DotArgs & a, hipStream_t s) { return launch_f32(false, fmt, a, s); }
int launch_dot_fast_f32(int fmt, const DotArgs & a, hipStream_t s) { return launch_f32(true, fmt, a, s); }

// ------------------------------------------------------------ decode ops --
__global__ void k_router_sel(const float * logits, uint32_t ntok, uint32_t n_expert,
                             uint32_t top_k, uint32_t norm, float scale,
                             uint32_t * ids, float * gates) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= ntok) return;
    const float * lg = logits + (size_t)t * n_expert;
    uint32_t * id = ids + (size_t)t * top_k;
    float * gt = gates + (size_t)t * top_k;
    float w[256];
    float mx = -1e30f, sum = 0.f, tsum = 0.f;
    for (uint32_t i = 0; i < n_expert; ++i) if (lg[i] > mx) mx = lg[i];
    for (uint32_t i = 0; i < n_expert; ++i) { w[i] = expf(lg[i] - mx); sum += w[i]; }
    for (uint32_t i = 0; i < n_expert; ++i) w[i] /= sum;
    for (uint32_t k = 0; k < top_k; ++k) {
        uint32_t best = 0;
        float bw = -1.f;
        for (uint32_t i = 0; i < n_expert; ++i) {
            bool taken = false;
            for (uint32_t k2 = 0; k2 < k; ++k2) if (id[k2] == i) { taken = true; break; }
            if (!taken && w[i] > bw) { bw = w[i]; best = i; }
        }
        id[k] = best; gt[k] = bw; tsum += bw;
    }
    for (uint32_t k = 0; k < top_k; ++k) {
        if (norm) gt[k] /= tsum;
        gt[k] *= scale;
    }
}

// One wave per token (n_expert <= 64, top_k <= 8): router_token_wave, the
// per-token form also run inside the fused router + grouped expert matvec.
__global__ __launch_bounds__(64) void k_router_wave(const float * logits, uint32_t n_expert, uint32_t top_k,
                                                    uint32_t norm, float scale, uint32_t * ids, float * gates) {
    const uint32_t t = blockIdx.x;
    router_token_wave(logits + (size_t)t * n_expert, n_expert, top_k, norm, scale, threadIdx.x,
                      ids + (size_t)t * top_k, gates + (size_t)t * top_k);
}

__global__ void k_silu_mul(const float * gate, const float * up, float * h, uint32_t n,
                           uint32_t gstride, uint32_t hstride) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x, c = blockIdx.y;
    if (i >= n) return;
    const float g = gate[(size_t)c * gstride + i];
    h[(size_t)c * hstride + i] = (g / (1.0f + expf(-g))) * up[(size_t)c * gstride + i];
}

__global__ void k_wmerge(const float * parts, const float * gates, const float * add1,
                         const float * add2, float * y, float scale, uint32_t n_parts,
                         uint32_t n, uint32_t n_full, uint32_t pstride, uint32_t ystride) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x, c = blockIdx.y;
    if (i >= n) return;
    const float * pc = parts + (size_t)c * pstride;
    const float * gc = gates ? gates + (size_t)c * (n_full > n_parts ? n_full : n_parts) : nullptr;
    float gsc = 1.0f;
    if (gc && n_full > n_parts) {
        float s = 0.f, sf = 0.f;
        for (uint32_t q = 0; q < n_parts; ++q) s += gc[q];
        for (uint32_t q = 0; q < n_full; ++q) sf += gc[q];
        if (s > 0.f) gsc = sf / s;
    }
    float acc = 0.f;
    for (uint32_t q = 0; q < n_parts; ++q)
        acc += (gc ? gsc * gc[q] : 1.0f) * pc[(size_t)q * n + i];
    acc *= scale;
    if (add1) acc += add1[(size_t)c * ystride + i];
    if (add2) acc += add2[(size_t)c * ystride + i];
    y[(size_t)c * ystride + i] = acc;
}

__global__ void k_merge(const float * x, float * y, uint32_t rows, uint32_t nparts) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows) return;
    float acc = 0.f;
    for (uint32_t p = 0; p < nparts; ++p) acc += x[(size_t)p * rows + i];
    y[i] = acc;
}

int launch_router_sel(const float * logits, uint32_t ntok, uint32_t n_expert, uint32_t top_k,
                      uint32_t norm, float scale, uint32_t * ids, float * gates, hipStream_t s) {
    if (n_expert == 0 || n_expert > 256 || top_k == 0 || top_k > n_expert)
        return set_error(FLH_ERR_ARG, "router_sel: need 0 < top_k <= n_expert <= 256");
    if (ntok == 0) return FLH_OK;
    if (n_expert <= 64 && top_k <= 8) {
        hipLaunchKernelGGL(k_router_wave, dim3(ntok), dim3(64), 0, s, logits, n_expert, top_k, norm, scale, ids,
                           gates);
        return hip_check(hipGetLastError(), "k_router_wave launch");
    }
    hipLaunchKernelGGL(k_router_sel, dim3((ntok + 63) / 64), dim3(64), 0, s, logits, ntok,
                       n_expert, top_k, norm, scale, ids, gates);
    return hip_check(hipGetLastError(), "k_router_sel launch");
}
int launch_silu_mul(const float * gate, const float * up, float * h, uint32_t n, uint32_t ncol,
                    uint32_t gstride, uint32_t hstride, hipStream_t s) {
    if (n == 0 || ncol == 0) return FLH_OK;
    hipLaunchKernelGGL(k_silu_mul, dim3((n + 255) / 256, ncol), dim3(256), 0, s, gate, up, h, n,
                       gstride, hstride);
    return hip_check(hipGetLastError(), "k_silu_mul launch");
}
int launch_wmerge(const float * parts, const float * gates, const float * add1, const float * add2,
                  float * y, float scale, uint32_t n_parts, uint32_t n, uint32_t n_full,
                  uint32_t ncol, uint32_t pstride, uint32_t ystride, hipStream_t s) {
    if (n == 0 || ncol == 0) return FLH_OK;
    hipLaunchKernelGGL(k_wmerge, dim3((n + 255) / 256, ncol), dim3(256), 0, s, parts, gates, add1,
                       add2, y, scale, n_parts, n, n_full, pstride, ystride);
    return hip_check(hipGetLastError(), "k_wmerge launch");
}
int launch_merge(const float * x, float * y, uint32_t rows, uint32_t nparts, hipStream_t s) {
    if (rows == 0) return FLH_OK;
    hipLaunchKernelGGL(k_merge, dim3((rows + 255) / 256), dim3(256), 0, s, x, y, rows, nparts);
    return hip_check(hipGetLastError(), "k_merge launch");
}

__global__ void k_zero(uint32_t * p, size_t nw, uint8_t * tail, uint32_t ntail) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < nw) p[i] = 0u;
    if (i < ntail) tail[i] = 0;
}
// zero n bytes with a kernel (no hipMemsetAsync: this may run inside a
// captured HIP graph).  p must be 4-byte aligned.
int launch_zero(void * p, size_t n, hipStream_t s) {
    if (n == 0) return FLH_OK;
    if ((uintptr_t)p & 3) return set_error(FLH_ERR_ARG, "zero: pointer must be 4-byte aligned");
    const size_t nw = n / 4;
    const uint32_t nt = (uint32_t)(n & 3);
    const size_t m = nw > nt ? nw : nt;
    hipLaunchKernelGGL(k_zero, dim3((uint32_t)((m + 255) / 256)), dim3(256), 0, s, (uint32_t *)p, nw,
                       (uint8_t *)p + nw * 4, nt);
    return hip_check(hipGetLastError(), "k_zero launch");
}

}  // namespace flh
