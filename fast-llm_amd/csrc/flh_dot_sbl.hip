// flh_dot_sbl.hip -- single-column row-dots with one superblock (Q4_K, Q6_K
// x q8_K) or four 32-weight blocks (Q8_0, Q5_0, IQ2_XXS, IQ3_XXS x q8_1) per
// lane, the routed (MoE) form of the same launch, its RMSNORM -> ACT_Q8
// prologue (NORM), and a several-column form for the 32-weight-block formats
// (k_dot_sbl_nx, at the end of this file).
//
// The streaming kernel of flh_dot_kstream.hip splits a superblock over four
// lanes, which costs every quarter its own scale decode, a DPP reduction and
// a parked term, and it folds each batch of rows after a workgroup barrier.
// For one activation column the work per superblock is small enough that the
// lane can take all of it:
//
//   * a CHUNK is rpc = floor(64 / P) whole rows (P lanes per row: nsb for the
//     K formats, 2 nsb for 32-weight blocks; row r = lane / P, position
//     lane % P); its bytes go HBM -> LDS in 16-byte direct-to-LDS loads, each
//     1 KiB request of a wave fully coalesced;
//   * a lane's activation block is the same for every chunk (its position),
//     so it is read once from the workgroup's staged copy into registers
//     (Q4_K: 256 int8, 8 sub-block sums, d: 73 VGPRs);
//   * the lane computes its superblock's exact integer partials and the
//     reference factors (Q4_K: iacc, imin with d*dk and -(dmin*dk),
//     fl_dot_i8k_q4_K, src/runtime/quants.h:538-561; Q6_K: iacc with d*dk,
//     :563-594); rows of 4, 8 or 16 superblocks fold in registers (the
//     accumulator chains run down the row's lanes by DPP row shifts), other
//     rows park the terms in a wave-local LDS area where lanes (row, k) run
//     accumulator k over its terms in the reference's fmaf order; then
//     (a0 + a1) + (a2 + a3) by DPP;
//   * waves are independent after the activation is staged: no barrier per
//     batch, each wave keeps two chunks in flight and refills a stage as soon
//     as its bytes are in registers.
//
// The 32-weight-block formats fold as fl_dot_i8_q8_0 (src/runtime/quants.h:
// 438-466): block b of a row goes to accumulator b & 3, so a lane holding
// blocks 4p .. 4p + 3 (position p) contributes one term to each accumulator.
// Terms are parked so that each (row, accumulator) chain is contiguous, and a
// fold lane reads 16 of them per LDS round trip.  Q5_0 lanes take 88
// contiguous bytes; IQ lanes take half a superblock (its d, the half's group
// data and, for IQ3, its sign words), with the codebook and a sign-mask table
// staged in LDS once per workgroup.
//
// Chunks are dealt to workgroups first (chunk c -> workgroup c % G), so a
// matrix with fewer chunks than waves still spreads over every CU.
// With FUSE (Q4_K), the workgroup quantises the fp32 column itself (ACT_Q8,
// src/runtime/quants.h:382-402): wave w takes superblocks w, w + W, ...; the
// staged bytes are the q8_K block's, and workgroup s % G also writes both
// appendices of superblock s, so memory ends up as after a separate ACT_Q8
// launch (with every appendix store in workgroup 0, that workgroup finished
// ~2 us after the others).  With NORM the items come from the input column
// with their norm weights and are normalised first (the sum of squares in the
// order of the standalone RMSNORM kernel), and the owning workgroup also
// stores y.
#include "flh_kstream.h"
#include "flh_internal.h"
#include "flh_status.h"
#include <algorithm>
#include <type_traits>

namespace flh {

// Development timing probe (compiled only with -DFLH_TRACE): per wave of
// the single-column kernel, s_memrealtime stamps at entry (0), after the
// activation barrier (1), when the first chunk has landed (2), when the last
// chunk has landed (3), at exit (4); slot 7 holds the chunk count.
#ifdef FLH_TRACE
__device__ uint64_t g_sbl_trace[4096 * 8 * 8];
#define SBL_STAMP(k) do { if (lane == 0 && blockIdx.x < 4096) \
    g_sbl_trace[((size_t)blockIdx.x * 8 + wave) * 8 + (k)] = __builtin_amdgcn_s_memrealtime(); } while (0)
extern "C" int flh_sbl_trace(uint64_t * host, size_t n) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_sbl_trace), n * 8, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -2;
}
extern "C" int flh_sbl_trace_clear(void) {
    static uint64_t zeros[4096 * 8 * 8];
    return hipMemcpyToSymbol(HIP_SYMBOL(g_sbl_trace), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice) == hipSuccess ? 0 : -2;
}
#else
#define SBL_STAMP(k) do { } while (0)
#endif

namespace {

constexpr uint32_t SBL_XS = 304;    // LDS bytes per staged q8_K block
// A staged block is the 292-byte q8_K block placed 12 bytes into its 304-byte
// slot: f32 d at +12, int16 bsums[16] at +16, int8 qs[256] at +48 (both
// 16-byte aligned).  304 = 76 dwords: 16 consecutive blocks start in 16
// distinct 4-bank groups, so lanes reading 16 positions do not conflict.

// s_waitcnt vmcnt(n) for a wave-uniform run-time n (clamped to 31: waiting
// for more loads than asked is always safe)
__device__ __forceinline__ void wait_vm_dyn(uint32_t n) {
    switch (n) {
#define FLH_WV(k) case k: WAIT_VM(k); break;
        FLH_WV(0) FLH_WV(1) FLH_WV(2) FLH_WV(3) FLH_WV(4) FLH_WV(5) FLH_WV(6) FLH_WV(7)
        FLH_WV(8) FLH_WV(9) FLH_WV(10) FLH_WV(11) FLH_WV(12) FLH_WV(13) FLH_WV(14) FLH_WV(15)
        FLH_WV(16) FLH_WV(17) FLH_WV(18) FLH_WV(19) FLH_WV(20) FLH_WV(21) FLH_WV(22) FLH_WV(23)
        FLH_WV(24) FLH_WV(25) FLH_WV(26) FLH_WV(27) FLH_WV(28) FLH_WV(29) FLH_WV(30)
#undef FLH_WV
        default: WAIT_VM(31); break;
    }
}

// the 144-byte Q4_K superblock at LDS address p as 9 x 16 bytes
__device__ __forceinline__ void lds_ld_q4k(const void * p, u32x4a (&v)[9]) {
    asm volatile("ds_read_b128 %0, %9\n\tds_read_b128 %1, %9 offset:16\n\tds_read_b128 %2, %9 offset:32\n\t"
                 "ds_read_b128 %3, %9 offset:48\n\tds_read_b128 %4, %9 offset:64\n\tds_read_b128 %5, %9 offset:80\n\t"
                 "ds_read_b128 %6, %9 offset:96\n\tds_read_b128 %7, %9 offset:112\n\tds_read_b128 %8, %9 offset:128\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
                   "=&v"(v[7]), "=&v"(v[8])
                 : "v"(lds_off(p)) : "memory");
}
// 16 bytes at LDS address p; the caller waits (lds_wait4) before any use
__device__ __forceinline__ u32x4a lds_ld128_nw(const void * p) {
    u32x4a v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(lds_off(p)) : "memory");
    return v;
}
__device__ __forceinline__ void lds_wait4(u32x4a & a, u32x4a & b, u32x4a & c, u32x4a & d) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) :: "memory");
}
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void lds_wait8(u32x4a (&t)[8]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5]), "+v"(t[6]), "+v"(t[7])
                 :: "memory");
}
__device__ __forceinline__ void lds_wait16(u32x4a (&t)[16]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5]), "+v"(t[6]), "+v"(t[7]),
                   "+v"(t[8]), "+v"(t[9]), "+v"(t[10]), "+v"(t[11]), "+v"(t[12]), "+v"(t[13]), "+v"(t[14]), "+v"(t[15])
                 :: "memory");
}
__device__ __forceinline__ void lds_st64(void * p, u32x2v v) {
    asm volatile("ds_write_b64 %0, %1" :: "v"(lds_off(p)), "v"(v));
}
__device__ __forceinline__ void lds_st16(void * p, uint32_t v) {
    asm volatile("ds_write_b16 %0, %1" :: "v"(lds_off(p)), "v"(v));
}
// global store kept out of the compiler's wait-count bookkeeping (the wave
// counts its own memory operations)
__device__ __forceinline__ void gst_x1(float * p, uint32_t v) {
    asm volatile("global_store_dword %0, %1, off" :: "v"(p), "v"(v) : "memory");
}

__device__ __forceinline__ u32x4a lds_ld128(const void * p) {
    u32x4a v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_off(p)) : "memory");
    return v;
}
// ACT_Q8's appendix bytes of one 256-element chunk (k_act_q8's lane code),
// (inlined once: the item loop stays rolled); one workgroup in G takes each chunk
__device__ __forceinline__ void write_appendices(const float (&v)[4], uint32_t lane, uint32_t chunk,
                                                           uint8_t * q81, uint8_t * q8k, uint32_t cols) {
    act_q8_lanes(v, lane, chunk, q81, q8k, cols);
}

// A lane's activation superblock: 64 dwords of int8, the 8 sub-block sums
// (bsums[2t] + bsums[2t+1]), and d.
struct XQ4 {
    u32x4a q[16];
    int b[8];
    float dk;
};

__device__ __forceinline__ void load_xq4(const uint8_t * xb, XQ4 & X) {
    u32x4a bs0, bs1;
    asm volatile("ds_read_b128 %0, %18 offset:48\n\tds_read_b128 %1, %18 offset:64\n\tds_read_b128 %2, %18 offset:80\n\t"
                 "ds_read_b128 %3, %18 offset:96\n\tds_read_b128 %4, %18 offset:112\n\tds_read_b128 %5, %18 offset:128\n\t"
                 "ds_read_b128 %6, %18 offset:144\n\tds_read_b128 %7, %18 offset:160\n\tds_read_b128 %8, %18 offset:176\n\t"
                 "ds_read_b128 %9, %18 offset:192\n\tds_read_b128 %10, %18 offset:208\n\tds_read_b128 %11, %18 offset:224\n\t"
                 "ds_read_b128 %12, %18 offset:240\n\tds_read_b128 %13, %18 offset:256\n\tds_read_b128 %14, %18 offset:272\n\t"
                 "ds_read_b128 %15, %18 offset:288\n\tds_read_b128 %16, %18 offset:16\n\tds_read_b128 %17, %18 offset:32\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(X.q[0]), "=&v"(X.q[1]), "=&v"(X.q[2]), "=&v"(X.q[3]), "=&v"(X.q[4]), "=&v"(X.q[5]),
                   "=&v"(X.q[6]), "=&v"(X.q[7]), "=&v"(X.q[8]), "=&v"(X.q[9]), "=&v"(X.q[10]), "=&v"(X.q[11]),
                   "=&v"(X.q[12]), "=&v"(X.q[13]), "=&v"(X.q[14]), "=&v"(X.q[15]), "=&v"(bs0), "=&v"(bs1)
                 : "v"(lds_off(xb)) : "memory");
    X.dk = __uint_as_float(lds_ld32(xb + 12));
    const uint32_t w[8] = {bs0.x, bs0.y, bs0.z, bs0.w, bs1.x, bs1.y, bs1.z, bs1.w};
#pragma unroll
    for (int t = 0; t < 8; ++t) X.b[t] = (int)(int16_t)(w[t] & 0xFFFFu) + (int)(int16_t)(w[t] >> 16);
}

// Exact integer partials of one Q4_K superblock against the lane's
// activation: iacc = sum_t sc_t * dot_t, imin = sum_t m_t * bsum_t.  Sub-block
// pair g holds sub-block 2g in the low nibbles of qs[32g..32g+31] and 2g+1 in
// the high nibbles.  Every product fits 24 bits (sc, m < 64; |dot| <= 60960;
// |bsum| <= 4064), so the multiplies are full-rate v_mul_i32_i24.
__device__ __forceinline__ void sbl_q4k(const u32x4a (&w)[9], const XQ4 & X, int & ia, int & im) {
    const u32x4a hd = w[0];
    const uint32_t sclo = hd.y & 0x3F3F3F3Fu, mlo = hd.z & 0x3F3F3F3Fu;
    const uint32_t schi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
    const uint32_t mhi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
    int acc = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const u32x4a qa = w[1 + 2 * g], qb = w[2 + 2 * g];
        const uint32_t Q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        const u32x4a xa = X.q[4 * g], xb = X.q[4 * g + 1], xc = X.q[4 * g + 2], xd = X.q[4 * g + 3];
        const uint32_t XL[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        const uint32_t XH[8] = {xc.x, xc.y, xc.z, xc.w, xd.x, xd.y, xd.z, xd.w};
        int dl[2] = {0, 0}, dh[2] = {0, 0};                     // two chains each (exact sums)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            dl[i & 1] = dot4((int)(Q[i] & 0x0F0F0F0Fu), (int)XL[i], dl[i & 1]);
            dh[i & 1] = dot4((int)((Q[i] >> 4) & 0x0F0F0F0Fu), (int)XH[i], dh[i & 1]);
        }
        const int dlo = dl[0] + dl[1], dhi = dh[0] + dh[1];
        const uint32_t scw = g < 2 ? sclo : schi, sh = 16 * (g & 1);
        acc += __mul24((int)((scw >> sh) & 0xFFu), dlo) + __mul24((int)((scw >> (sh + 8)) & 0xFFu), dhi);
    }
    int mi = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) mi += __mul24((int)(((t < 4 ? mlo : mhi) >> (8 * (t & 3))) & 0xFFu), X.b[t]);
    ia = acc;
    im = mi;
}

// ---- Q6_K: a lane takes one 210-byte superblock (ql[128], qh[64], int8
// scales[16], d), 2-byte aligned in LDS: 54 dwords are read from the aligned
// address below and shifted into place (W[i] = bytes 4i .. 4i + 3).
__device__ __forceinline__ void lds_ld_q6k(uint32_t p, uint32_t (&W)[53]) {
    const uint32_t a4 = p & ~3u, sh = p & 3u;
    u32x2v R[27];
    asm volatile("ds_read2_b32 %0, %27 offset1:1\n\tds_read2_b32 %1, %27 offset0:2 offset1:3\n\t"
                 "ds_read2_b32 %2, %27 offset0:4 offset1:5\n\tds_read2_b32 %3, %27 offset0:6 offset1:7\n\t"
                 "ds_read2_b32 %4, %27 offset0:8 offset1:9\n\tds_read2_b32 %5, %27 offset0:10 offset1:11\n\t"
                 "ds_read2_b32 %6, %27 offset0:12 offset1:13\n\tds_read2_b32 %7, %27 offset0:14 offset1:15\n\t"
                 "ds_read2_b32 %8, %27 offset0:16 offset1:17\n\tds_read2_b32 %9, %27 offset0:18 offset1:19\n\t"
                 "ds_read2_b32 %10, %27 offset0:20 offset1:21\n\tds_read2_b32 %11, %27 offset0:22 offset1:23\n\t"
                 "ds_read2_b32 %12, %27 offset0:24 offset1:25\n\tds_read2_b32 %13, %27 offset0:26 offset1:27\n\t"
                 "ds_read2_b32 %14, %27 offset0:28 offset1:29\n\tds_read2_b32 %15, %27 offset0:30 offset1:31\n\t"
                 "ds_read2_b32 %16, %27 offset0:32 offset1:33\n\tds_read2_b32 %17, %27 offset0:34 offset1:35\n\t"
                 "ds_read2_b32 %18, %27 offset0:36 offset1:37\n\tds_read2_b32 %19, %27 offset0:38 offset1:39\n\t"
                 "ds_read2_b32 %20, %27 offset0:40 offset1:41\n\tds_read2_b32 %21, %27 offset0:42 offset1:43\n\t"
                 "ds_read2_b32 %22, %27 offset0:44 offset1:45\n\tds_read2_b32 %23, %27 offset0:46 offset1:47\n\t"
                 "ds_read2_b32 %24, %27 offset0:48 offset1:49\n\tds_read2_b32 %25, %27 offset0:50 offset1:51\n\t"
                 "ds_read2_b32 %26, %27 offset0:52 offset1:53\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(R[0]), "=&v"(R[1]), "=&v"(R[2]), "=&v"(R[3]), "=&v"(R[4]), "=&v"(R[5]), "=&v"(R[6]),
                   "=&v"(R[7]), "=&v"(R[8]), "=&v"(R[9]), "=&v"(R[10]), "=&v"(R[11]), "=&v"(R[12]), "=&v"(R[13]),
                   "=&v"(R[14]), "=&v"(R[15]), "=&v"(R[16]), "=&v"(R[17]), "=&v"(R[18]), "=&v"(R[19]),
                   "=&v"(R[20]), "=&v"(R[21]), "=&v"(R[22]), "=&v"(R[23]), "=&v"(R[24]), "=&v"(R[25]), "=&v"(R[26])
                 : "v"(a4) : "memory");
#pragma unroll
    for (int i = 0; i < 53; ++i) {
        const uint32_t lo = (i & 1) ? R[i >> 1].y : R[i >> 1].x;
        const uint32_t hi = ((i + 1) & 1) ? R[(i + 1) >> 1].y : R[(i + 1) >> 1].x;
        W[i] = alignb(hi, lo, sh);
    }
}

// A lane's activation superblock for Q6_K: 64 dwords of int8, the 16
// sub-block sums (int16 bsums), and d.
struct XQ6 {
    u32x4a q[16];
    int bs[16];
    float dk;
};

__device__ __forceinline__ void load_xq6(const uint8_t * xb, XQ6 & X) {
    XQ4 t;
    load_xq4(xb, t);                                              // the int8 and d
#pragma unroll
    for (int i = 0; i < 16; ++i) X.q[i] = t.q[i];
    X.dk = t.dk;
    const u32x4a b0 = lds_ld128(xb + 16), b1 = lds_ld128(xb + 32);
    const uint32_t w[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int t2 = 0; t2 < 8; ++t2) {
        X.bs[2 * t2] = (int)(int16_t)(w[t2] & 0xFFFFu);
        X.bs[2 * t2 + 1] = (int)(int16_t)(w[t2] >> 16);
    }
}

// Exact iacc of one Q6_K superblock (fl_dot_i8k_q6_K, src/runtime/quants.h:
// 563-594): sum over the 16 sub-blocks of sc_i * (idot_i - 32 * bsum_i), as
// sum sc_i * idot_i - 32 * sum sc_i * bsum_i.  Element 128h + 32g + l takes
// the low (g < 2) or high nibble of ql[64h + 32(g & 1) + l] and bits 2g, 2g + 1
// of qh[32h + l]; every product fits 24 bits (|idot| <= 16 * 63 * 128).
__device__ __forceinline__ int sbl_q6k(const uint32_t (&W)[53], const XQ6 & X) {
    int dsum[16];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                int sa = 0;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int j = 4 * k + jj;
                    const uint32_t ql = W[16 * h + 8 * (g & 1) + j], qh = W[32 + 8 * h + j];
                    const uint32_t v = ((g < 2 ? ql : ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * g)) & 0x03030303u) << 4);
                    const int xi = 32 * h + 8 * g + j;
                    const u32x4a xq = X.q[xi >> 2];
                    const uint32_t xv = (xi & 3) == 0 ? xq.x : (xi & 3) == 1 ? xq.y : (xi & 3) == 2 ? xq.z : xq.w;
                    sa = dot4((int)v, (int)xv, sa);
                }
                dsum[8 * h + 2 * g + k] = sa;
            }
    int acc = 0, bacc = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int sc = (int)(int8_t)((W[48 + (i >> 2)] >> (8 * (i & 3))) & 0xFFu);
        acc += __mul24(sc, dsum[i]);
        bacc += __mul24(sc, X.bs[i]);
    }
    return acc - 32 * bacc;
}

// ---- Q8_0: a lane takes half of a 256-weight unit, 4 blocks of 34 bytes
// (136 bytes, 8-byte aligned); the activation's q8_1 blocks are staged as
// 48-byte slots (d at +12, the 32 int8 at +16, 16-byte aligned).
constexpr uint32_t SBL_X8 = 48;
typedef u32x2v u32x2a;

// the lane's 136 bytes at LDS address p as 34 dwords
__device__ __forceinline__ void lds_ld_q8h(const void * p, uint32_t (&d)[34]) {
    u32x2a v[17];
    asm volatile("ds_read_b64 %0, %17\n\tds_read_b64 %1, %17 offset:8\n\tds_read_b64 %2, %17 offset:16\n\t"
                 "ds_read_b64 %3, %17 offset:24\n\tds_read_b64 %4, %17 offset:32\n\tds_read_b64 %5, %17 offset:40\n\t"
                 "ds_read_b64 %6, %17 offset:48\n\tds_read_b64 %7, %17 offset:56\n\tds_read_b64 %8, %17 offset:64\n\t"
                 "ds_read_b64 %9, %17 offset:72\n\tds_read_b64 %10, %17 offset:80\n\tds_read_b64 %11, %17 offset:88\n\t"
                 "ds_read_b64 %12, %17 offset:96\n\tds_read_b64 %13, %17 offset:104\n\tds_read_b64 %14, %17 offset:112\n\t"
                 "ds_read_b64 %15, %17 offset:120\n\tds_read_b64 %16, %17 offset:128\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
                   "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]), "=&v"(v[12]), "=&v"(v[13]),
                   "=&v"(v[14]), "=&v"(v[15]), "=&v"(v[16])
                 : "v"(lds_off(p)) : "memory");
#pragma unroll
    for (int i = 0; i < 17; ++i) { d[2 * i] = v[i].x; d[2 * i + 1] = v[i].y; }
}

// A lane's four q8_1 blocks: 32 dwords of int8 and the four d.
struct XQ8 {
    u32x4a q[8];
    float dx[4];
};

__device__ __forceinline__ void load_xq8(const uint8_t * xb, XQ8 & X) {
    asm volatile("ds_read_b128 %0, %8 offset:16\n\tds_read_b128 %1, %8 offset:32\n\tds_read_b128 %2, %8 offset:64\n\t"
                 "ds_read_b128 %3, %8 offset:80\n\tds_read_b128 %4, %8 offset:112\n\tds_read_b128 %5, %8 offset:128\n\t"
                 "ds_read_b128 %6, %8 offset:160\n\tds_read_b128 %7, %8 offset:176\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(X.q[0]), "=&v"(X.q[1]), "=&v"(X.q[2]), "=&v"(X.q[3]), "=&v"(X.q[4]), "=&v"(X.q[5]),
                   "=&v"(X.q[6]), "=&v"(X.q[7])
                 : "v"(lds_off(xb)) : "memory");
#pragma unroll
    for (int m = 0; m < 4; ++m) X.dx[m] = h2f(lds_ld32(xb + SBL_X8 * m + 12) & 0xFFFFu);
}

// Exact block dots and reference factors (fl_dot_i8_q8_0,
// src/runtime/quants.h:438-447: fmaf(d_w * d_x, (float)idot, a4[b & 3])) of
// the lane's four blocks.  Block m starts at byte 34m: its d is the low half
// of dword 0 (m = 0), the high half of dword 8, the low half of dword 17 or
// the high half of dword 25; the int8 of blocks 1 and 3 are dword aligned,
// those of blocks 0 and 2 start two bytes into a dword.
__device__ __forceinline__ void sbl_q8_0(const uint32_t (&D)[34], const XQ8 & X, float (&f)[4], int (&id)[4]) {
    const uint32_t dw[4] = {D[0] & 0xFFFFu, D[8] >> 16, D[17] & 0xFFFFu, D[25] >> 16};
    const int q0[4] = {0, 9, 17, 26};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const u32x4a xa = X.q[2 * m], xb = X.q[2 * m + 1];
        const uint32_t XV[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t q = (m & 1) ? D[q0[m] + i] : alignb(D[q0[m] + i + 1], D[q0[m] + i], 2);
            if (i & 1) s1 = dot4((int)q, (int)XV[i], s1); else s0 = dot4((int)q, (int)XV[i], s0);
        }
        id[m] = s0 + s1;
        f[m] = h2f(dw[m]) * X.dx[m];
    }
}

// ---- Q5_0: a lane takes 4 blocks of 22 bytes (88 bytes, 8-byte aligned).
__device__ __forceinline__ void lds_ld_q5h(const void * p, uint32_t (&d)[22]) {
    u32x2a v[11];
    asm volatile("ds_read_b64 %0, %11\n\tds_read_b64 %1, %11 offset:8\n\tds_read_b64 %2, %11 offset:16\n\t"
                 "ds_read_b64 %3, %11 offset:24\n\tds_read_b64 %4, %11 offset:32\n\tds_read_b64 %5, %11 offset:40\n\t"
                 "ds_read_b64 %6, %11 offset:48\n\tds_read_b64 %7, %11 offset:56\n\tds_read_b64 %8, %11 offset:64\n\t"
                 "ds_read_b64 %9, %11 offset:72\n\tds_read_b64 %10, %11 offset:80\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
                   "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10])
                 : "v"(lds_off(p)) : "memory");
#pragma unroll
    for (int i = 0; i < 11; ++i) { d[2 * i] = v[i].x; d[2 * i + 1] = v[i].y; }
}

// Block dots of fl_dot_i8_q5_0 (src/runtime/quants.h:449-466): the unshifted
// 5-bit values (0..31) against the q8_1 quants, minus 16 x the block's
// activation sum; factor d_w * d_x.  Block m starts at byte 22m: blocks 0 and
// 2 at a dword boundary (d, then qh 2 bytes into it, nibbles 6 bytes in),
// blocks 1 and 3 two bytes into dword 5 / 16 (qh and the nibbles aligned).
__device__ __forceinline__ void sbl_q5_0(const uint32_t (&D)[22], const XQ8 & X, const int (&xsum)[4], float (&f)[4],
                                         int (&id)[4]) {
    const int o[4] = {0, 5, 11, 16};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const bool odd = m & 1;
        const uint32_t db = odd ? D[o[m]] >> 16 : D[o[m]] & 0xFFFFu;
        const uint32_t qh = odd ? D[o[m] + 1] : alignb(D[o[m] + 1], D[o[m]], 2);
        const u32x4a xa = X.q[2 * m], xb = X.q[2 * m + 1];
        const uint32_t XV[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q = odd ? D[o[m] + 2 + k] : alignb(D[o[m] + 2 + k], D[o[m] + 1 + k], 2);
            const uint32_t lo = (q & 0x0F0F0F0Fu) | (spread4((qh >> (4 * k)) & 0xFu) << 4);
            const uint32_t hi = ((q >> 4) & 0x0F0F0F0Fu) | (spread4((qh >> (16 + 4 * k)) & 0xFu) << 4);
            s0 = dot4((int)lo, (int)XV[k], s0);
            s1 = dot4((int)hi, (int)XV[4 + k], s1);
        }
        id[m] = s0 + s1 - 16 * xsum[m];
        f[m] = h2f(db) * X.dx[m];
    }
}

// ---- IQ2_XXS / IQ3_XXS: a lane takes half a superblock, groups 4h .. 4h + 3
// (h = lane & 1) of superblock lane >> 1.  Its bytes are not contiguous:
// d at the superblock's start, the half's 32 bytes of group data at +2 + 32h
// (IQ2: per group 4 grid indices and the scale/sign word w1; IQ3: 8 grid
// indices per group) and, for IQ3, the half's four w1 words at +66 + 16h.
// Superblocks are 66 / 98 bytes, so these pieces are 2-byte aligned: they
// are read as dwords from the aligned address below and shifted into place.
template <int FMT>
__device__ __forceinline__ void lds_ld_iqh(const uint8_t * st, uint32_t lane, uint32_t & db, uint32_t (&G)[8],
                                           uint32_t (&S)[4]) {
    constexpr uint32_t BB = iq_block_bytes(FMT);
    const uint32_t base = lds_off(st) + BB * (lane >> 1), h = lane & 1u;
    const uint32_t A = base + 2 + 32 * h, a4 = A & ~3u, sh = A & 3u;
    u32x2a r0, r1, r2, r3;
    uint32_t r4, dv;
    asm volatile("ds_read_u16 %5, %6\n\tds_read2_b32 %0, %7 offset1:1\n\tds_read2_b32 %1, %7 offset0:2 offset1:3\n\t"
                 "ds_read2_b32 %2, %7 offset0:4 offset1:5\n\tds_read2_b32 %3, %7 offset0:6 offset1:7\n\t"
                 "ds_read_b32 %4, %7 offset:32\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3), "=&v"(r4), "=&v"(dv)
                 : "v"(base), "v"(a4) : "memory");
    const uint32_t w[9] = {r0.x, r0.y, r1.x, r1.y, r2.x, r2.y, r3.x, r3.y, r4};
#pragma unroll
    for (int k = 0; k < 8; ++k) G[k] = alignb(w[k + 1], w[k], sh);
    db = dv;
    if constexpr (FMT == FMT_IQ3_XXS) {
        const uint32_t s4 = (A + 64 - 16 * h) & ~3u;              // same alignment as A
        u32x2a t0, t1;
        uint32_t t2;
        asm volatile("ds_read2_b32 %0, %3 offset1:1\n\tds_read2_b32 %1, %3 offset0:2 offset1:3\n\t"
                     "ds_read_b32 %2, %3 offset:16\n\ts_waitcnt lgkmcnt(0)"
                     : "=&v"(t0), "=&v"(t1), "=&v"(t2) : "v"(s4) : "memory");
        const uint32_t u[5] = {t0.x, t0.y, t1.x, t1.y, t2};
#pragma unroll
        for (int k = 0; k < 4; ++k) S[k] = alignb(u[k + 1], u[k], sh);
    }
}

// Grid entries (magnitude bytes) of the lane's four groups, all requested in
// one LDS round trip: E[4m + l] = run l of group m as (elements 0-3,
// elements 4-7).  IQ2: one 8-byte entry per index byte of w0 (G[2m]); IQ3:
// one 4-byte entry per index byte of G[2m], G[2m + 1].
template <int FMT>
__device__ __forceinline__ void iq_runs(uint32_t grid, const uint32_t (&G)[8], u32x2a (&E)[16]) {
    if constexpr (FMT == FMT_IQ2_XXS) {
        uint32_t ad[16];
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int l = 0; l < 4; ++l) ad[4 * m + l] = grid + 8 * ((G[2 * m] >> (8 * l)) & 0xFFu);
        asm volatile("ds_read_b64 %0, %16\n\tds_read_b64 %1, %17\n\tds_read_b64 %2, %18\n\tds_read_b64 %3, %19\n\t"
                     "ds_read_b64 %4, %20\n\tds_read_b64 %5, %21\n\tds_read_b64 %6, %22\n\tds_read_b64 %7, %23\n\t"
                     "ds_read_b64 %8, %24\n\tds_read_b64 %9, %25\n\tds_read_b64 %10, %26\n\tds_read_b64 %11, %27\n\t"
                     "ds_read_b64 %12, %28\n\tds_read_b64 %13, %29\n\tds_read_b64 %14, %30\n\tds_read_b64 %15, %31\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(E[0]), "=&v"(E[1]), "=&v"(E[2]), "=&v"(E[3]), "=&v"(E[4]), "=&v"(E[5]), "=&v"(E[6]),
                       "=&v"(E[7]), "=&v"(E[8]), "=&v"(E[9]), "=&v"(E[10]), "=&v"(E[11]), "=&v"(E[12]), "=&v"(E[13]),
                       "=&v"(E[14]), "=&v"(E[15])
                     : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(ad[4]), "v"(ad[5]), "v"(ad[6]), "v"(ad[7]),
                       "v"(ad[8]), "v"(ad[9]), "v"(ad[10]), "v"(ad[11]), "v"(ad[12]), "v"(ad[13]), "v"(ad[14]),
                       "v"(ad[15])
                     : "memory");
    } else {
        uint32_t ad[32], v[32];
#pragma unroll
        for (int b = 0; b < 32; ++b) ad[b] = grid + 4 * ((G[b >> 2] >> (8 * (b & 3))) & 0xFFu);
        asm volatile("ds_read_b32 %0, %32\n\tds_read_b32 %1, %33\n\tds_read_b32 %2, %34\n\tds_read_b32 %3, %35\n\t"
                     "ds_read_b32 %4, %36\n\tds_read_b32 %5, %37\n\tds_read_b32 %6, %38\n\tds_read_b32 %7, %39\n\t"
                     "ds_read_b32 %8, %40\n\tds_read_b32 %9, %41\n\tds_read_b32 %10, %42\n\tds_read_b32 %11, %43\n\t"
                     "ds_read_b32 %12, %44\n\tds_read_b32 %13, %45\n\tds_read_b32 %14, %46\n\tds_read_b32 %15, %47\n\t"
                     "ds_read_b32 %16, %48\n\tds_read_b32 %17, %49\n\tds_read_b32 %18, %50\n\tds_read_b32 %19, %51\n\t"
                     "ds_read_b32 %20, %52\n\tds_read_b32 %21, %53\n\tds_read_b32 %22, %54\n\tds_read_b32 %23, %55\n\t"
                     "ds_read_b32 %24, %56\n\tds_read_b32 %25, %57\n\tds_read_b32 %26, %58\n\tds_read_b32 %27, %59\n\t"
                     "ds_read_b32 %28, %60\n\tds_read_b32 %29, %61\n\tds_read_b32 %30, %62\n\tds_read_b32 %31, %63\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
                       "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]), "=&v"(v[12]), "=&v"(v[13]),
                       "=&v"(v[14]), "=&v"(v[15]), "=&v"(v[16]), "=&v"(v[17]), "=&v"(v[18]), "=&v"(v[19]),
                       "=&v"(v[20]), "=&v"(v[21]), "=&v"(v[22]), "=&v"(v[23]), "=&v"(v[24]), "=&v"(v[25]),
                       "=&v"(v[26]), "=&v"(v[27]), "=&v"(v[28]), "=&v"(v[29]), "=&v"(v[30]), "=&v"(v[31])
                     : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(ad[4]), "v"(ad[5]), "v"(ad[6]), "v"(ad[7]),
                       "v"(ad[8]), "v"(ad[9]), "v"(ad[10]), "v"(ad[11]), "v"(ad[12]), "v"(ad[13]), "v"(ad[14]),
                       "v"(ad[15]), "v"(ad[16]), "v"(ad[17]), "v"(ad[18]), "v"(ad[19]), "v"(ad[20]), "v"(ad[21]),
                       "v"(ad[22]), "v"(ad[23]), "v"(ad[24]), "v"(ad[25]), "v"(ad[26]), "v"(ad[27]), "v"(ad[28]),
                       "v"(ad[29]), "v"(ad[30]), "v"(ad[31])
                     : "memory");
#pragma unroll
        for (int k = 0; k < 16; ++k) E[k] = u32x2a{v[2 * k], v[2 * k + 1]};
    }
}

// Negation masks of the lane's 16 runs (sign field l of group m's w1) from
// the 128-entry table at LDS address tab (entry s7: the byte masks of
// iq_sign8(s7)'s bits 0-3 and 4-7), in one LDS round trip.
__device__ __forceinline__ void iq_negs(uint32_t tab, const uint32_t (&w1)[4], u32x2a (&N)[16]) {
    uint32_t ad[16];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int l = 0; l < 4; ++l) ad[4 * m + l] = tab + 8 * ((w1[m] >> (7 * l)) & 127u);
    asm volatile("ds_read_b64 %0, %16\n\tds_read_b64 %1, %17\n\tds_read_b64 %2, %18\n\tds_read_b64 %3, %19\n\t"
                 "ds_read_b64 %4, %20\n\tds_read_b64 %5, %21\n\tds_read_b64 %6, %22\n\tds_read_b64 %7, %23\n\t"
                 "ds_read_b64 %8, %24\n\tds_read_b64 %9, %25\n\tds_read_b64 %10, %26\n\tds_read_b64 %11, %27\n\t"
                 "ds_read_b64 %12, %28\n\tds_read_b64 %13, %29\n\tds_read_b64 %14, %30\n\tds_read_b64 %15, %31\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(N[0]), "=&v"(N[1]), "=&v"(N[2]), "=&v"(N[3]), "=&v"(N[4]), "=&v"(N[5]), "=&v"(N[6]),
                   "=&v"(N[7]), "=&v"(N[8]), "=&v"(N[9]), "=&v"(N[10]), "=&v"(N[11]), "=&v"(N[12]), "=&v"(N[13]),
                   "=&v"(N[14]), "=&v"(N[15])
                 : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(ad[4]), "v"(ad[5]), "v"(ad[6]), "v"(ad[7]),
                   "v"(ad[8]), "v"(ad[9]), "v"(ad[10]), "v"(ad[11]), "v"(ad[12]), "v"(ad[13]), "v"(ad[14]),
                   "v"(ad[15])
                 : "memory");
}

// Group dots of the codebook formats: the signed grid magnitudes (run l takes
// sign field l of w1, bit j negating element 8l + j) against the q8_1 quants;
// factor db * d_x with db = (d * (0.5 + s)) * 0.25 (IQ2) or * 0.5 (IQ3), s =
// w1 >> 28 (kernels_gpu.h:759-852; fold as fl_dot_i8_q8_0).
template <int FMT>
__device__ __forceinline__ void sbl_iq(const uint8_t * st, uint32_t lane, uint32_t grid, const XQ8 & X, float (&f)[4],
                                       int (&id)[4]) {
    uint32_t dbits, G[8], S[4];
    lds_ld_iqh<FMT>(st, lane, dbits, G, S);
    uint32_t w1s[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) w1s[m] = FMT == FMT_IQ2_XXS ? G[2 * m + 1] : S[m];
    u32x2a E[16], N[16];
    iq_runs<FMT>(grid, G, E);
    iq_negs(grid + 2048, w1s, N);
    const float d = h2f(dbits);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const uint32_t w1 = w1s[m];
        const u32x4a xa = X.q[2 * m], xb = X.q[2 * m + 1];
        const uint32_t XV[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            s0 = dot4((int)iq_apply(E[4 * m + l].x, N[4 * m + l].x), (int)XV[2 * l], s0);
            s1 = dot4((int)iq_apply(E[4 * m + l].y, N[4 * m + l].y), (int)XV[2 * l + 1], s1);
        }
        id[m] = s0 + s1;
        f[m] = iq_db(FMT, d, w1) * X.dx[m];
    }
}

}  // namespace

// One pass over all rows for one column.  Launch: G workgroups of W waves,
// dynamic LDS = W * 2 * slot (rings) + the staged activation (rounded to
// 1 KiB) + W * (TB + 256) bytes (fold terms and old y values) + the IQ
// codebook (2 KiB).
//
// MOE: one token's routed experts (ROUTER_SEL fused or ids given):
// blockIdx.y is the (token, slot) pair p, whose y is m.y + p * ystride and
// whose activation is column p (per-slot x) or the token's; the pair's
// expert is known only after routing, so its weight requests wait for that,
// while the y and activation DMAs go out first.
//
// H = 2 (32-weight-block formats, rows of more than 64 four-block halves):
// a lane takes the halves l and l + PL of its row (PL = lanes of a row; the
// lanes' reads stay one half apart, as with H = 1), decoding them one after
// the other against their own activation blocks and parking each half's
// terms at its own position of the chains, so the fold reads the same chains
// in the same order as with one half per lane.
template <int FMT, bool FUSE, int W, bool MOE = false, bool NORM = false, int H = 1>
__global__ __launch_bounds__(64 * W) void k_dot_sbl(DotArgs a, uint32_t rpc, uint32_t ni, uint32_t slot, uint32_t pre,
                                                    MoeArgs m, NormArgs nm) {
    static_assert(!NORM || (FUSE && (W == 4 || W == 8)), "RMSNORM rides on the fused quantisation, 16 % W == 0");
    static_assert(FMT == FMT_Q4_K || !FUSE, "only Q4_K fuses the quantisation");
    static_assert(H == 1 || (H == 2 && FMT != FMT_Q4_K && FMT != FMT_Q6_K && !FUSE),
                  "two halves per lane: unfused 32-weight-block formats");
    static_assert(FMT != FMT_Q6_K || !MOE, "Q6_K experts run on the grouped streaming kernel");
    static_assert(!MOE || !FUSE, "the routed launch reads a ready appendix");
    static_assert(FMT == FMT_Q4_K || FMT == FMT_Q6_K || FMT == FMT_Q8_0 || FMT == FMT_Q5_0 ||
                  FMT == FMT_IQ2_XXS || FMT == FMT_IQ3_XXS, "a K format or a 32-weight-block format");
    constexpr bool Q6 = FMT == FMT_Q6_K;
    constexpr bool Q8 = FMT != FMT_Q4_K && !Q6;                   // 4 blocks of 32 weights per lane
    constexpr bool IQ = FMT == FMT_IQ2_XXS || FMT == FMT_IQ3_XXS;
    // bytes of a lane's weights (IQ: half a superblock's share)
    constexpr uint32_t B = FMT == FMT_Q4_K ? 144 : Q6 ? 210 : FMT == FMT_Q8_0 ? 136 : FMT == FMT_Q5_0 ? 88
                                                 : iq_block_bytes(FMT) / 2;
    constexpr uint32_t TB = Q8 ? 4096 : 1024;                     // fold-term bytes of a wave
    extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
    const uint32_t nsb = a.cols >> 8, rows = a.rows, cols = a.cols;
    const uint32_t P = Q8 ? 2 * nsb : nsb;                        // lane shares (fold terms) of a row
    const uint32_t PL = P / H;                                    // lanes of a row
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const uint32_t C = (rows + rpc - 1) / rpc;                    // chunks of the matrix
    const uint32_t first = b + G * wave, stride = G * W;          // this wave's chunks: first + stride * i
    const uint32_t nck = first < C ? (C - first + stride - 1) / stride : 0u;
    uint8_t * ring = sm + (size_t)wave * 2 * slot;
    uint8_t * xs = sm + (size_t)W * 2 * slot;
    const uint32_t xs_bytes = ((Q8 ? nsb * 8 * SBL_X8 : nsb * SBL_XS) + 1023u) & ~1023u;
    uint8_t * T = xs + xs_bytes + wave * (TB + 256);              // fold terms of this wave
    uint8_t * Y = T + TB;                                         // [64] old y values of this wave
    const uint32_t grid = lds_off(xs + xs_bytes + W * (TB + 256)); // IQ codebook (2 KiB), sign masks (1 KiB)
    if constexpr (MOE) {
        const uint32_t p = blockIdx.y;
        a.x = m.x + (size_t)(m.x_per_slot ? p : p / m.top_k) * m.xstride;
        a.y = m.y + (size_t)p * m.ystride;
    }
    const uint8_t * w = MOE ? m.w : a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0);
    const uint64_t cb = (uint64_t)rpc * P * B;                    // bytes of a full chunk
    const uint8_t * xk = (const uint8_t *)a.x + xqk_off(cols);
    uint32_t ops = 0;                                             // memory operations issued by this wave
    SBL_STAMP(0);

    // Old y values (y += semantics) of up to ypc chunks go to Y by a DMA:
    // word l holds row l % rpc of chunk l / rpc.  Issued first, so every
    // later wait covers it.
    const uint32_t ypc = 64u / rpc;
    const uint32_t yi = lane / rpc, yr = lane - yi * rpc;
    auto yload = [&](uint32_t grp) {
        const uint32_t i = grp * ypc + yi;
        const uint32_t row = (first + stride * i) * rpc + yr;
        const bool v = yi < ypc && i < nck && row < rows;
        __builtin_amdgcn_global_load_lds(GPTR(a.y + (v ? row : 0u)), LPTR(Y), 4, 0, 0);
        ++ops;
    };
    yload(0);
    uint32_t y_mark = ops;
    if constexpr (IQ) {
        // the codebook (IQ2 2 KiB, IQ3 1 KiB) by wave 0, covered by its
        // activation wait and the barrier after it
        constexpr uint32_t GB = FMT == FMT_IQ2_XXS ? 2048 : 1024;
        const uint8_t * gsrc = FMT == FMT_IQ2_XXS ? (const uint8_t *)k_iq2_grid : (const uint8_t *)k_iq3_grid;
        if (wave == 0) {
            for (uint32_t t = 0; t < GB / 1024; ++t) {
                __builtin_amdgcn_global_load_lds(GPTR(gsrc + 1024 * t + 16 * lane),
                                                 LPTR(xs + xs_bytes + W * (TB + 256) + 1024 * t), 16, 0, 0);
                ++ops;
            }
        }
        // sign-mask table after it (published by the staging barrier)
        if (tid < 128) {
            const uint32_t sg = iq_sign8(tid);
            lds_st64(xs + xs_bytes + W * (TB + 256) + 2048 + 8 * tid, u32x2a{iq_neg4(sg), iq_neg4(sg >> 4)});
        }
    }

    // activation: DMA of the q8_K blocks into the staged layout, or (FUSE)
    // of the fp32 superblocks w, w + W, ... of this wave into its second
    // ring stage (its first chunk is requested after the quantisation)
    const uint32_t nfi = FUSE ? (nsb > wave ? (nsb - wave + W - 1) / W : 0u) : 0u;   // <= 8 (host check)
    if constexpr (FUSE) {
        // NORM: the input column instead, and the norm weights of the same
        // superblocks after it (nfi <= 4, host check)
        const float * xsrc = NORM ? nm.x : a.x;
        for (uint32_t j = 0; j < nfi; ++j) {
            __builtin_amdgcn_global_load_lds(GPTR(xsrc + 256 * (wave + W * j) + 4 * lane), LPTR(ring + slot + 1024 * j),
                                             16, 0, 0);
            ++ops;
            if constexpr (NORM) {
                __builtin_amdgcn_global_load_lds(GPTR(nm.wn + 256 * (wave + W * j) + 4 * lane),
                                                 LPTR(ring + slot + 1024 * (4 + j)), 16, 0, 0);
                ++ops;
            }
        }
    } else if constexpr (Q8) {
        // q8_1 block j as three 16-byte pieces starting 12 bytes early (the
        // bytes before block 0 belong to the fp32 column): slot j of 48 bytes
        const uint8_t * x1 = (const uint8_t *)a.x + xq_off(cols);
        const uint32_t NP = nsb * 8 * 3, nxi = (NP + 63) / 64;
        for (uint32_t t = wave; t < nxi; t += W) {
            const uint32_t j = 64 * t + lane, jj = j < NP ? j : NP - 1;
            const uint32_t blk = jj / 3, i = jj - 3 * blk;
            __builtin_amdgcn_global_load_lds(GPTR(x1 + 36 * blk + 16 * i - 12), LPTR(xs + 1024 * t), 16, 0, 0);
            ++ops;
        }
    } else {
        const uint32_t NP = nsb * 19, nxi = (NP + 63) / 64;
        for (uint32_t t = wave; t < nxi; t += W) {
            const uint32_t j = 64 * t + lane, jj = j < NP ? j : NP - 1;
            const uint32_t s = jj / 19, i = jj - 19 * s;
            __builtin_amdgcn_global_load_lds(GPTR(xk + 292 * s + 16 * i - 12), LPTR(xs + 1024 * t), 16, 0, 0);
            ++ops;
        }
    }
    const uint32_t x_mark = ops;
    if constexpr (MOE) {
        // the pair's expert (routing waits for every load issued so far,
        // which the activation wait below needs anyway)
        __shared__ uint32_t rids[256];
        const uint32_t * ids = moe_route(m, rids);
        const uint32_t e = ids[blockIdx.y];
        if (e >= m.n_expert) {                                    // nothing routed to this pair
            WAIT_VM(0);                                           // no DMA may land after exit
            return;
        }
        w += (size_t)e * m.estride;
    }
    // Every wave's activation requests enter the CU's memory queue before any
    // weight request: served in order, they would otherwise wait behind the
    // CU's whole initial weight burst (~150 KB, several us at a CU's share of
    // HBM bandwidth), and no wave could start before the last one.
    __builtin_amdgcn_s_barrier();

    // weight prologue: chunks 0 and (unless the stage holds fp32 x) 1
    uint32_t mark[2] = {0u, 0u};
    auto issue = [&](uint32_t i, uint8_t * st) {
        const uint32_t c = first + stride * i;
        const uint8_t * g = w + (uint64_t)c * cb;
        const uint32_t nrow = min(rpc, rows - c * rpc);
        const uint32_t vb = nrow * P * B;                         // valid bytes (a multiple of 16)
        for (uint32_t t = 0; t < ni; ++t) {
            const uint32_t o = 1024 * t + 16 * lane;
            __builtin_amdgcn_global_load_lds(GPTR(g + (o < vb ? o : vb - 16)), LPTR(st + 1024 * t), 16, 0, FLH_KS_AUX);
        }
        ops += ni;
    };
    // Only waves below `pre` request a chunk before the activation has
    // landed: the activation's own requests queue chip-wide behind whatever
    // the launch has asked for (a 37 MB initial burst delays them by ~4 us).
    const bool early = wave < pre;
    if (early && nck > 0) { issue(0, ring); mark[0] = ops; }

    // wait for this wave's activation loads alone
    wait_vm_dyn(ops - x_mark);
    SBL_STAMP(5);
    if constexpr (FUSE) {
        uint8_t * q81 = (uint8_t *)a.x + xq_off(cols);
        uint8_t * q8k = (uint8_t *)a.x + xqk_off(cols);
        const uint8_t * xf = ring + slot + 16 * lane;
        // Two items per pass, loop kept rolled (unrolled with the appendix
        // writer inlined it was ~16 KB of code, run once per wave).  The two
        // items' maxima share one reduction: v_permlane32_swap leaves item
        // a's partials in lanes 0-31 and item b's in lanes 32-63, DPP and
        // v_permlane16_swap finish both, and one division sequence gives both
        // scales (each lane's values are computed exactly as for one item).
        // Every workgroup quantises the whole column: VALU throughput, 2
        // waves per SIMD x 2 items at 4096 columns.
        auto store_item = [&](const float (&v)[4], uint32_t s, float d, float id) {
            const uint32_t pk = quant4(v, id);
            const int s16 = sum4i(dot4((int)pk, 0x01010101, 0));     // 16-element block sum
            uint8_t * xb = xs + SBL_XS * s;
            lds_st32(xb + 48 + 4 * lane, pk);
            if ((lane & 3) == 0) lds_st16(xb + 16 + 2 * (lane >> 2), (uint32_t)s16);
            if (lane == 0) lds_st32(xb + 12, __float_as_uint(d));
            if (s % G == b) {                                     // each block by one workgroup
                if constexpr (NORM) *(float4 *)((float *)a.x + 256 * s + 4 * lane) = make_float4(v[0], v[1], v[2], v[3]);
                write_appendices(v, lane, s, q81, q8k, cols);
            }
        };
        // NORM: the sum of squares in k_rmsnorm_act_q8_reg's order.  Its
        // thread (v, l) sums elements 4l .. 4l + 3 of superblocks v, v + 16,
        // ... in turn, a butterfly makes the 64-lane total of "wave" v, and
        // every thread adds the 16 totals in order.  Here superblock s sits in
        // wave s % W (W divides 16), so wave w holds the partials of v = w +
        // W q, q < 16 / W, for its items j = q, q + 16 / W, ... (nfi <= 4).
        float nrm_s = 0.f;
        if constexpr (NORM) {
            __shared__ __attribute__((aligned(16))) float nparts[16];
            constexpr uint32_t NQ = 16 / W;
            float ss[NQ];
#pragma unroll
            for (uint32_t q = 0; q < NQ; ++q) ss[q] = 0.f;
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                if (j < nfi) {
                    const u32x4a r = lds_ld128(xf + 1024 * j);
                    const float x0 = __uint_as_float(r.x), x1 = __uint_as_float(r.y);
                    const float x2 = __uint_as_float(r.z), x3 = __uint_as_float(r.w);
                    float & t = ss[j % NQ];
                    t += x0 * x0;
                    t += x1 * x1;
                    t += x2 * x2;
                    t += x3 * x3;
                }
            }
            // the butterfly ss += (value of lane ^ o), o = 1, 2, ..., 32
            // (xor_lane: the values of __shfl_xor without LDS round trips)
#pragma unroll
            for (uint32_t q = 0; q < NQ; ++q) {
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) ss[q] += xor_lane(ss[q], o, lane);
                if (lane == 0) lds_st32(&nparts[wave + W * q], __float_as_uint(ss[q]));
            }
            lds_barrier();                                        // (no wait for the weight DMAs)
            u32x4a p0 = lds_ld128_nw(&nparts[0]), p1 = lds_ld128_nw(&nparts[4]);
            u32x4a p2 = lds_ld128_nw(&nparts[8]), p3 = lds_ld128_nw(&nparts[12]);
            lds_wait4(p0, p1, p2, p3);                            // one LDS round trip for the 16 totals
            const uint32_t pv[16] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w,
                                     p2.x, p2.y, p2.z, p2.w, p3.x, p3.y, p3.z, p3.w};
            float tn = 0.f;
#pragma unroll
            for (int v = 0; v < 16; ++v) tn += __uint_as_float(pv[v]);
            nrm_s = 1.0f / sqrtf(tn / (float)cols + nm.eps);
        }
        // y = (x * s) * wn of the lane's 4 elements (NORM), in place
        auto normed = [&](float (&v)[4], uint32_t j) {
            if constexpr (NORM) {
                const u32x4a wr = lds_ld128(xf + 1024 * (4 + j));
                const float wv[4] = {__uint_as_float(wr.x), __uint_as_float(wr.y), __uint_as_float(wr.z),
                                     __uint_as_float(wr.w)};
#pragma unroll
                for (int k = 0; k < 4; ++k) v[k] = v[k] * nrm_s * wv[k];
            }
        };
#pragma unroll 1
        for (uint32_t j = 0; j < nfi; j += 2) {
            const bool two = j + 1 < nfi;                         // wave-uniform
            const uint32_t sa = wave + W * j;
            u32x4a ra = lds_ld128_nw(xf + 1024 * j), rb = lds_ld128_nw(xf + 1024 * (two ? j + 1 : j));
            u32x4a r2 = ra, r3 = rb;
            lds_wait4(ra, rb, r2, r3);
            float va[4] = {__uint_as_float(ra.x), __uint_as_float(ra.y), __uint_as_float(ra.z), __uint_as_float(ra.w)};
            float vb[4] = {__uint_as_float(rb.x), __uint_as_float(rb.y), __uint_as_float(rb.z), __uint_as_float(rb.w)};
            normed(va, j);
            normed(vb, two ? j + 1 : j);
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(absmax4(va)), __float_as_uint(absmax4(vb)),
                                                             false, false);
            uint32_t m = umax8(max((uint32_t)sw[0], (uint32_t)sw[1]));
            m = max(m, (uint32_t)rmir((int)m));                   // each 16-lane row
            const auto rs = __builtin_amdgcn_permlane16_swap(m, m, false, false);
            const float amax = __uint_as_float(max((uint32_t)rs[0], (uint32_t)rs[1]));   // a: lanes 0-31, b: 32-63
            const float dv = amax / 127.f;
            const float iv = amax > 0.f ? 127.f / amax : 0.f;
            store_item(va, sa, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dv), 0)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(iv), 0)));
            if (two)
                store_item(vb, sa + W, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dv), 32)),
                           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(iv), 32)));
        }
    }
    SBL_STAMP(6);
    lds_barrier();
    SBL_STAMP(1);
    typename std::conditional<Q8, XQ8, typename std::conditional<Q6, XQ6, XQ4>::type>::type X;
    int xsum[H][4] = {};                                          // Q5_0: the blocks' activation sums
    XQ8 X2;                                                       // H = 2: the second half's blocks
    (void)X2;
    if constexpr (Q8) load_xq8(xs + 4 * SBL_X8 * (lane % PL), X);
    else if constexpr (Q6) load_xq6(xs + SBL_XS * (lane % nsb), X);
    else load_xq4(xs + SBL_XS * (lane % nsb), X);
    if constexpr (H == 2) load_xq8(xs + 4 * SBL_X8 * (lane % PL + PL), X2);
    if constexpr (FMT == FMT_Q5_0) {
#pragma unroll
        for (int h = 0; h < H; ++h)
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const XQ8 & XH = h ? X2 : X;
                const u32x4a xa = XH.q[2 * m], xb = XH.q[2 * m + 1];
                int t = 0;
                t = dot4(0x01010101, (int)xa.x, t); t = dot4(0x01010101, (int)xa.y, t);
                t = dot4(0x01010101, (int)xa.z, t); t = dot4(0x01010101, (int)xa.w, t);
                t = dot4(0x01010101, (int)xb.x, t); t = dot4(0x01010101, (int)xb.y, t);
                t = dot4(0x01010101, (int)xb.z, t); t = dot4(0x01010101, (int)xb.w, t);
                xsum[h][m] = t;
            }
    }
    // The rest of the prologue comes after the barrier: a request blocks its
    // wave while the CU's memory queue is full, and a wave stuck there would
    // hold the whole workgroup at the barrier.
    if (!early && nck > 0) { issue(0, ring); mark[0] = ops; }
    // (FUSE: the second stage's fp32 reads are done, lds_wait4)
    if (nck > 1) { issue(1, ring + slot); mark[1] = ops; }

    const uint32_t fr = lane >> 2, fk = lane & 3;                 // fold lane: row r0 + fr, accumulator fk
    // K-format rows of 4, 8 or 16 superblocks fold in registers (DPP)
    const bool dppf = !Q8 && (nsb == 4 || nsb == 8 || nsb == 16);
    for (uint32_t i = 0; i < nck; ++i) {
        const uint32_t sl = i & 1u;
        uint8_t * st = ring + sl * slot;
        const uint32_t il = i % ypc;
        if (il == 0 && i != 0) {                                  // the next group's old y values
            yload(i / ypc);                                       // (the previous group's reads are done)
            y_mark = ops;
        }
        wait_vm_dyn(ops - mark[sl]);
        if (i == 0) SBL_STAMP(2);
        if (i + 1 == nck) SBL_STAMP(3);
        if constexpr (Q8) {
            const uint32_t r = lane / PL, pos = lane - r * PL;
            // H = 2: a lane past the chunk's rows decodes the first share
            // (its terms are not parked) instead of reading past the chunk
            const uint32_t ql = H == 2 && r >= rpc ? 0u : lane;
            float f[H][4];
            int id[H][4];
#pragma unroll
            for (int h = 0; h < H; ++h) {
                const uint32_t vl = ql + h * PL;                  // the lane's share of the chunk (rpc == 1 if H == 2)
                const XQ8 & XH = h ? X2 : X;
                if constexpr (FMT == FMT_Q8_0) {
                    uint32_t D[34];
                    lds_ld_q8h(st + B * vl, D);
                    sbl_q8_0(D, XH, f[h], id[h]);
                } else if constexpr (FMT == FMT_Q5_0) {
                    uint32_t D[22];
                    lds_ld_q5h(st + B * vl, D);
                    sbl_q5_0(D, XH, xsum[h], f[h], id[h]);
                } else {
                    sbl_iq<FMT>(st, vl, grid, XH, f[h], id[h]);
                }
            }
            if (i + 2 < nck) {                                    // refill this stage
                issue(i + 2, st);
                mark[sl] = ops;
            }
            // chain (row r, accumulator k) = its P terms in share order,
            // CS bytes per chain (16 bytes of padding spread the fold
            // lanes' reads over the banks)
            const uint32_t CS = 8 * P + 16;
            if (r < rpc) {
#pragma unroll
                for (int h = 0; h < H; ++h)
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        lds_st64(T + (4 * r + k) * CS + 8 * (pos + h * PL),
                                 u32x2a{__float_as_uint(f[h][k]), __float_as_uint((float)id[h][k])});
            }
        } else {
            // Q4_K: terms (d * dk) * iacc and -(dmin * dk) * imin; Q6_K:
            // (d * dk) * iacc, its second product -0.0 * 0 (adding it leaves
            // every value, signed zeros included, unchanged)
            int ia, im = 0;
            float f1, f2 = -0.f;
            if constexpr (Q6) {
                uint32_t W6[53];
                lds_ld_q6k(lds_off(st) + B * lane, W6);
                ia = sbl_q6k(W6, X);
                f1 = h2f(W6[52] & 0xFFFFu) * X.dk;
            } else {
                u32x4a wv[9];
                lds_ld_q4k(st + B * lane, wv);
                sbl_q4k(wv, X, ia, im);
                f1 = h2f(wv[0].x & 0xFFFFu) * X.dk;
                f2 = -(h2f(wv[0].x >> 16) * X.dk);
            }
            if (i + 2 < nck) {                                    // refill this stage
                issue(i + 2, st);
                mark[sl] = ops;
            }
            if (dppf) {
                // Rows of 4, 8 or 16 lanes sit inside one 16-lane DPP row:
                // accumulator k runs down positions k, k + 4, ... by shifting
                // the partial chain four lanes per step; after nsb / 4 steps
                // the row's last four lanes hold a0..a3.
                const float fi = (float)ia, fm = (float)im;
                auto term = [&](float prev) { return Q6 ? fmaf(f1, fi, prev) : fmaf(f2, fm, fmaf(f1, fi, prev)); };
                float acc = term(0.f);
                for (uint32_t q = 4; q < nsb; q += 4) {
                    const float prev = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x114,
                                                                                  0xF, 0xF, false));
                    acc = term(prev);
                }
                const float s01 = acc + qx1f(acc);
                const float tot = s01 + qx2f(s01);
                if (il == 0) wait_vm_dyn(ops - y_mark);           // this group's old y values have landed
                const uint32_t r = lane / nsb;
                const float yo = __uint_as_float(lds_ld32(Y + 4 * ((il * rpc + r) & 63u)));
                const uint32_t row0 = (first + stride * i) * rpc, row = row0 + r;
                if (lane - r * nsb == nsb - 4 && row < rows) gst_x1(a.y + row, __float_as_uint(yo + tot));
                ++ops;                                            // lane nsb - 4 (row 0 of the chunk) stores
                continue;
            }
            // one row per chunk (more than 32 superblocks): accumulator k's
            // terms (positions k, k + 4, ...) contiguous; else lane order
            const u32x4a tv{__float_as_uint(f1), __float_as_uint((float)ia), __float_as_uint(f2),
                            __float_as_uint((float)im)};
            if (rpc == 1) {
                if (lane < nsb) lds_st128(T + (lane & 3) * (16 * ((nsb + 3) >> 2)) + 16 * (lane >> 2), tv);
            } else {
                lds_st128(T + 16 * lane, tv);
            }
        }
        // reference fold: accumulator fk of row r0 + fr over its terms in
        // order (Q4_K: positions fk, fk + 4, ...; Q8_0: block fk of every
        // lane of the row), 16 rows per pass
        if (il == 0) wait_vm_dyn(ops - y_mark);                   // this group's old y values have landed
        for (uint32_t r0 = 0; r0 < rpc; r0 += 16) {
            const uint32_t r = r0 + fr;
            float acc = 0.f;
            if (Q8 && r < rpc) {
                // 16 terms (8 x 16 bytes) per LDS round trip; P is even
                const uint8_t * tr = T + (4 * r + fk) * (8 * P + 16);
                for (uint32_t j0 = 0; j0 < P; j0 += 16) {
                    u32x4a t[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) t[q] = lds_ld128_nw(tr + 8 * (j0 + 2 * q < P ? j0 + 2 * q : j0));
                    lds_wait8(t);
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        if (j0 + 2 * q < P) {
                            acc = fmaf(__uint_as_float(t[q].x), __uint_as_float(t[q].y), acc);
                            acc = fmaf(__uint_as_float(t[q].z), __uint_as_float(t[q].w), acc);
                        }
                    }
                }
            } else if (rpc == 1) {
                if (lane < 4) {                                   // one LDS round trip (<= 16 terms)
                    const uint32_t nk = (nsb - fk + 3) >> 2;      // nsb > 32: 9 .. 16 terms
                    const uint8_t * tr = T + fk * (16 * ((nsb + 3) >> 2));
                    u32x4a t[16];
#pragma unroll
                    for (int q = 0; q < 16; ++q) t[q] = lds_ld128_nw(tr + 16 * (q < (int)nk ? q : 0));
                    lds_wait16(t);
#pragma unroll
                    for (int q = 0; q < 16; ++q) {
                        if (q < (int)nk) {
                            acc = fmaf(__uint_as_float(t[q].x), __uint_as_float(t[q].y), acc);
                            acc = fmaf(__uint_as_float(t[q].z), __uint_as_float(t[q].w), acc);
                        }
                    }
                }
            } else if (r < rpc) {
                const uint8_t * tr = T + 16 * (r * nsb);
                for (uint32_t j0 = fk; j0 < nsb; j0 += 16) {
                    u32x4a t0 = lds_ld128_nw(tr + 16 * j0);
                    u32x4a t1 = lds_ld128_nw(tr + 16 * (j0 + 4 < nsb ? j0 + 4 : j0));
                    u32x4a t2 = lds_ld128_nw(tr + 16 * (j0 + 8 < nsb ? j0 + 8 : j0));
                    u32x4a t3 = lds_ld128_nw(tr + 16 * (j0 + 12 < nsb ? j0 + 12 : j0));
                    lds_wait4(t0, t1, t2, t3);
                    const u32x4a tt[4] = {t0, t1, t2, t3};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (j0 + 4 * q < nsb) {
                            acc = fmaf(__uint_as_float(tt[q].x), __uint_as_float(tt[q].y), acc);
                            acc = fmaf(__uint_as_float(tt[q].z), __uint_as_float(tt[q].w), acc);
                        }
                    }
                }
            }
            const float s01 = acc + qx1f(acc);
            const float tot = s01 + qx2f(s01);
            const float yo = __uint_as_float(lds_ld32(Y + 4 * ((il * rpc + r) & 63u)));
            const uint32_t row0 = (first + stride * i) * rpc + r0, row = row0 + fr;
            if (r < rpc && fk == 0 && row < rows) gst_x1(a.y + row, __float_as_uint(yo + tot));
            ops += row0 < rows ? 1u : 0u;                         // lane 0 stores iff row r0 exists
        }
    }
    WAIT_VM(0);
    SBL_STAMP(4);
#ifdef FLH_TRACE
    if (lane == 0 && blockIdx.x < 4096) g_sbl_trace[((size_t)blockIdx.x * 8 + wave) * 8 + 7] = nck;
#endif
}

// LDS of the several-column kernel: quants [NX][8 nsb][32], d words [NX][8 nsb]
// (each rounded to 1 KiB: the staging DMAs write whole 1 KiB / 256 B rows),
// per wave CG * rpc * 4 parked chains of 8 P + 16 bytes and 2 x 64 old y values
__host__ __device__ inline uint32_t sbl_nx_xq_bytes(uint32_t NX, uint32_t nsb) { return (NX * nsb * 256 + 1023) & ~1023u; }
__host__ __device__ inline uint32_t sbl_nx_xd_bytes(uint32_t NX, uint32_t nsb) { return (NX * nsb * 32 + 1023) & ~1023u; }
__host__ __device__ inline uint32_t sbl_nx_tw(uint32_t CG, uint32_t rpc, uint32_t P) { return CG * rpc * 4 * (8 * P + 16) + 512; }

// ---- several activation columns (32-weight-block formats) -----------------
//
// The lane layout of the single-column kernel (4 blocks of a row per lane),
// with the weights decoded once per chunk into 32 int8 words and 4 weight
// factors, then dotted with each column in turn.  The columns' q8_1 blocks
// are staged as quants [NX][8][P][16 B] (piece q = 2 m + h of position
// pos: half h of block 4 pos + m, so the lanes' reads of one piece are
// adjacent and conflict-free) and the (d, s) words [NX][8 nsb]; a lane reads
// its 128 quant bytes and 4 d of a column with one LDS round trip.  Terms (f, (float) idot) are parked per (column, row,
// accumulator) chain for up to 4 columns at a time and folded as in the
// single-column kernel: every column's output is the single-column result,
// bit for bit (fl_dot_i8_q8_0 / _q5_0, src/runtime/quants.h:438-466; the IQ
// factors of kernels_gpu.h:759-852).

// Weights of the lane's 4 blocks as int8 words Q[8m + i] (the element order
// of the q8_1 quants they meet) and factors wf[m] (the fp16 scale, or the IQ
// group scale); Q5_0 values are the unshifted 5-bit ones (0..31).
template <int FMT>
__device__ __forceinline__ void nx_decode(const uint8_t * st, uint32_t lane, uint32_t grid, uint32_t (&Q)[32],
                                          float (&wf)[4]) {
    if constexpr (FMT == FMT_Q8_0) {
        uint32_t D[34];
        lds_ld_q8h(st + 136 * lane, D);
        const uint32_t dw[4] = {D[0] & 0xFFFFu, D[8] >> 16, D[17] & 0xFFFFu, D[25] >> 16};
        const int q0[4] = {0, 9, 17, 26};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                Q[8 * m + i] = (m & 1) ? D[q0[m] + i] : alignb(D[q0[m] + i + 1], D[q0[m] + i], 2);
            wf[m] = h2f(dw[m]);
        }
    } else if constexpr (FMT == FMT_Q5_0) {
        uint32_t D[22];
        lds_ld_q5h(st + 88 * lane, D);
        const int o[4] = {0, 5, 11, 16};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const bool odd = m & 1;
            const uint32_t db = odd ? D[o[m]] >> 16 : D[o[m]] & 0xFFFFu;
            const uint32_t qh = odd ? D[o[m] + 1] : alignb(D[o[m] + 1], D[o[m]], 2);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t q = odd ? D[o[m] + 2 + k] : alignb(D[o[m] + 2 + k], D[o[m] + 1 + k], 2);
                Q[8 * m + k] = (q & 0x0F0F0F0Fu) | (spread4((qh >> (4 * k)) & 0xFu) << 4);
                Q[8 * m + 4 + k] = ((q >> 4) & 0x0F0F0F0Fu) | (spread4((qh >> (16 + 4 * k)) & 0xFu) << 4);
            }
            wf[m] = h2f(db);
        }
    } else {
        uint32_t dbits, G[8], S[4];
        lds_ld_iqh<FMT>(st, lane, dbits, G, S);
        uint32_t w1s[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) w1s[m] = FMT == FMT_IQ2_XXS ? G[2 * m + 1] : S[m];
        u32x2a E[16], N[16];
        iq_runs<FMT>(grid, G, E);
        iq_negs(grid + 2048, w1s, N);
        const float d = h2f(dbits);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                Q[8 * m + 2 * l] = iq_apply(E[4 * m + l].x, N[4 * m + l].x);
                Q[8 * m + 2 * l + 1] = iq_apply(E[4 * m + l].y, N[4 * m + l].y);
            }
            wf[m] = iq_db(FMT, d, w1s[m]);
        }
    }
}

// one column's quants of the lane (8 pieces of 16 bytes, piece q at
// xq + q * qs) and its 4 d words (at xd), requested together; nx_wait_col
// waits for them (the registers stay untouched in between)
__device__ __forceinline__ void nx_issue_col(const uint8_t * xq, uint32_t qs, const uint8_t * xd, u32x4a (&q)[8],
                                             u32x4a & dv) {
    const uint32_t a0 = lds_off(xq);
    asm volatile("ds_read_b128 %0, %9\n\tds_read_b128 %1, %10\n\tds_read_b128 %2, %11\n\tds_read_b128 %3, %12\n\t"
                 "ds_read_b128 %4, %13\n\tds_read_b128 %5, %14\n\tds_read_b128 %6, %15\n\tds_read_b128 %7, %16\n\t"
                 "ds_read_b128 %8, %17"
                 : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3]), "=&v"(q[4]), "=&v"(q[5]), "=&v"(q[6]),
                   "=&v"(q[7]), "=&v"(dv)
                 : "v"(a0), "v"(a0 + qs), "v"(a0 + 2 * qs), "v"(a0 + 3 * qs), "v"(a0 + 4 * qs), "v"(a0 + 5 * qs),
                   "v"(a0 + 6 * qs), "v"(a0 + 7 * qs), "v"(lds_off(xd))
                 : "memory");
}
__device__ __forceinline__ void nx_wait_col(u32x4a (&q)[8], u32x4a & dv) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]), "+v"(q[5]), "+v"(q[6]), "+v"(q[7]),
                   "+v"(dv)
                 :: "memory");
}

template <int FMT, int W, int CG>
__global__ __launch_bounds__(64 * W) void k_dot_sbl_nx(DotArgs a, uint32_t rpc, uint32_t ni, uint32_t slot, uint32_t pre,
                                                       uint32_t NX, uint32_t dep) {
    static_assert(FMT == FMT_Q8_0 || FMT == FMT_Q5_0 || FMT == FMT_IQ2_XXS || FMT == FMT_IQ3_XXS,
                  "a 32-weight-block format");
    constexpr bool IQ = FMT == FMT_IQ2_XXS || FMT == FMT_IQ3_XXS;
    constexpr uint32_t B = FMT == FMT_Q8_0 ? 136 : FMT == FMT_Q5_0 ? 88 : iq_block_bytes(FMT) / 2;
    extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
    const uint32_t nsb = a.cols >> 8, rows = a.rows, cols = a.cols, nx = a.nx;
    const uint32_t P = 2 * nsb, NB = 8 * nsb;                     // lanes of a row, q8_1 blocks of a column
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const uint32_t C = (rows + rpc - 1) / rpc;
    const uint32_t first = b + G * wave, stride = G * W;
    const uint32_t nck = first < C ? (C - first + stride - 1) / stride : 0u;
    // ring of dep (1 or 2) stages: a stage is free again once the lane's
    // decode has its bytes in registers
    uint8_t * ring = sm + (size_t)wave * dep * slot;
    uint8_t * xq = sm + (size_t)W * dep * slot;
    const uint32_t xqb = sbl_nx_xq_bytes(NX, nsb);
    uint8_t * xd = xq + xqb;
    const uint32_t CS = 8 * P + 16;                               // bytes per parked chain
    const uint32_t TW = sbl_nx_tw(CG, rpc, P);
    uint8_t * base = xd + sbl_nx_xd_bytes(NX, nsb);
    uint8_t * T = base + (size_t)wave * TW;
    uint8_t * Y = T + (size_t)CG * rpc * 4 * CS;                  // [2][64] old y values
    const uint32_t grid = lds_off(base + (size_t)W * TW);         // IQ codebook (2 KiB), sign masks (1 KiB)
    const uint64_t cb = (uint64_t)rpc * P * B;
    const uint8_t * w = a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0);
    auto x1 = [&](uint32_t p) -> const uint8_t * {
        return (const uint8_t *)(a.x + (size_t)(p < nx ? p : 0) * a.xstride) + xq_off(cols);
    };
    uint32_t ops = 0;

    // old y values of chunk i: word p * rpc + r = row r of column p (NX * rpc <= 64)
    uint32_t y_mark[2] = {0u, 0u};
    auto yload = [&](uint32_t i) {
        const uint32_t p = lane / rpc, r = lane - p * rpc;
        const uint32_t row = (first + stride * i) * rpc + r;
        const bool v = p < nx && row < rows;
        __builtin_amdgcn_global_load_lds(GPTR(v ? a.y + (size_t)p * a.ystride + row : a.y), LPTR(Y + 256 * (i & 1)),
                                         4, 0, 0);
        y_mark[i & 1] = ++ops;
    };
    if (nck > 0) yload(0);
    if constexpr (IQ) {
        constexpr uint32_t GB = FMT == FMT_IQ2_XXS ? 2048 : 1024;
        const uint8_t * gsrc = FMT == FMT_IQ2_XXS ? (const uint8_t *)k_iq2_grid : (const uint8_t *)k_iq3_grid;
        if (wave == 0) {
            for (uint32_t t = 0; t < GB / 1024; ++t) {
                __builtin_amdgcn_global_load_lds(GPTR(gsrc + 1024 * t + 16 * lane), LPTR(base + (size_t)W * TW + 1024 * t),
                                                 16, 0, 0);
                ++ops;
            }
        }
        if (tid < 128) {
            const uint32_t sg = iq_sign8(tid);
            lds_st64(base + (size_t)W * TW + 2048 + 8 * tid, u32x2a{iq_neg4(sg), iq_neg4(sg >> 4)});
        }
    }
    // activations: piece e = (p * 8 + q) * P + pos of the quants is half
    // q & 1 (16 bytes from byte 4 of the 36-byte q8_1 block) of column p's
    // block 4 pos + (q >> 1); the (d, s) word of block j at xd + 4 (p NB + j)
    {
        const uint32_t NQ = NX * NB * 2, nqi = (NQ + 63) / 64;
        for (uint32_t t = wave; t < nqi; t += W) {
            const uint32_t e = 64 * t + lane;
            if (e < NQ) {
                const uint32_t pq = e / P, pos = e - pq * P, p = pq >> 3, q = pq & 7u;
                __builtin_amdgcn_global_load_lds(GPTR(x1(p) + 36 * (4 * pos + (q >> 1)) + 4 + 16 * (q & 1)),
                                                 LPTR(xq + 1024 * t), 16, 0, 0);
            }
            ++ops;
        }
        const uint32_t ND = NX * NB, ndi = (ND + 63) / 64;
        for (uint32_t t = wave; t < ndi; t += W) {
            const uint32_t e = 64 * t + lane;
            if (e < ND) {
                const uint32_t p = e / NB;
                __builtin_amdgcn_global_load_lds(GPTR(x1(p) + 36 * (e - p * NB)), LPTR(xd + 256 * t), 4, 0, 0);
            }
            ++ops;
        }
    }
    const uint32_t x_mark = ops;
    __builtin_amdgcn_s_barrier();

    uint32_t mark[2] = {0u, 0u};
    auto issue = [&](uint32_t i, uint8_t * st) {
        const uint32_t c = first + stride * i;
        const uint8_t * g = w + (uint64_t)c * cb;
        const uint32_t nrow = min(rpc, rows - c * rpc);
        const uint32_t vb = nrow * P * B;                         // valid bytes (a multiple of 16)
        for (uint32_t t = 0; t < ni; ++t) {
            const uint32_t o = 1024 * t + 16 * lane;
            __builtin_amdgcn_global_load_lds(GPTR(g + (o < vb ? o : vb - 16)), LPTR(st + 1024 * t), 16, 0, FLH_KS_AUX);
        }
        ops += ni;
    };
    const bool early = wave < pre;
    if (early && nck > 0) { issue(0, ring); mark[0] = ops; }
    wait_vm_dyn(ops - x_mark);                                    // this wave's activation loads
    lds_barrier();                                                // everyone's
    if (!early && nck > 0) { issue(0, ring); mark[0] = ops; }
    if (dep == 2 && nck > 1) { issue(1, ring + slot); mark[1] = ops; }

    const uint32_t r = lane / P, pos = lane - r * P;              // the lane's row in a chunk, its position
    for (uint32_t i = 0; i < nck; ++i) {
        const uint32_t sl = dep == 2 ? (i & 1u) : 0u;
        uint8_t * st = ring + sl * slot;
        wait_vm_dyn(ops - mark[sl]);
        if (i + 1 < nck) yload(i + 1);
        uint32_t Q[32];
        float wf[4];
        nx_decode<FMT>(st, lane, grid, Q, wf);
        if (i + dep < nck) {                                      // refill this stage
            issue(i + dep, st);
            mark[sl] = ops;
        }
        const uint32_t row0 = (first + stride * i) * rpc;
        // columns g0 .. g0 + CG - 1 parked, then folded
        for (uint32_t g0 = 0; g0 < nx; g0 += CG) {
            if (r < rpc) {
                // column pl + 1's pieces are requested before column pl's dots
                u32x4a qa[8], da, qb[8], db;
                auto issue_col = [&](uint32_t pl, u32x4a (&q)[8], u32x4a & dv) {
                    nx_issue_col(xq + 16 * ((size_t)(g0 + pl) * 8 * P + pos), 16 * P,
                                 xd + 4 * ((size_t)(g0 + pl) * NB + 4 * pos), q, dv);
                };
                issue_col(0, qa, da);
#pragma unroll
                for (uint32_t pl = 0; pl < CG; ++pl) {
                    u32x4a (&q)[8] = (pl & 1) ? qb : qa;
                    u32x4a & dv = (pl & 1) ? db : da;
                    nx_wait_col(q, dv);
                    if (pl + 1 < CG) {
                        if (pl & 1) issue_col(pl + 1, qa, da);
                        else issue_col(pl + 1, qb, db);
                    }
                    const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        const uint32_t XV[8] = {q[2 * m].x, q[2 * m].y, q[2 * m].z, q[2 * m].w,
                                                q[2 * m + 1].x, q[2 * m + 1].y, q[2 * m + 1].z, q[2 * m + 1].w};
                        int s = 0, xs = 0;
#pragma unroll
                        for (int k = 0; k < 8; ++k) {
                            s = dot4((int)Q[8 * m + k], (int)XV[k], s);
                            if constexpr (FMT == FMT_Q5_0) xs = dot4(0x01010101, (int)XV[k], xs);
                        }
                        if constexpr (FMT == FMT_Q5_0) s -= 16 * xs;
                        const float f = wf[m] * h2f(dw[m] & 0xFFFFu);
                        lds_st64(T + ((pl * rpc + r) * 4 + m) * CS + 8 * pos,
                                 u32x2a{__float_as_uint(f), __float_as_uint((float)s)});
                    }
                }
            }
            if (g0 == 0) wait_vm_dyn(ops - y_mark[i & 1]);        // this chunk's old y values have landed
            // chain c = (pl * rpc + rr) * 4 + k: accumulator k of row rr,
            // column g0 + pl, over its P terms in position order
            const uint32_t nch = CG * rpc * 4;
            for (uint32_t c0 = 0; c0 < nch; c0 += 64) {
                const uint32_t c = c0 + lane, ch = c < nch ? c : nch - 1;
                const uint8_t * tr = T + ch * CS;
                float acc = 0.f;
                for (uint32_t j0 = 0; j0 < P; j0 += 16) {
                    u32x4a t[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) t[q] = lds_ld128_nw(tr + 8 * (j0 + 2 * q < P ? j0 + 2 * q : j0));
                    lds_wait8(t);
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        if (j0 + 2 * q < P) {
                            acc = fmaf(__uint_as_float(t[q].x), __uint_as_float(t[q].y), acc);
                            acc = fmaf(__uint_as_float(t[q].z), __uint_as_float(t[q].w), acc);
                        }
                    }
                }
                const float s01 = acc + qx1f(acc);
                const float tot = s01 + qx2f(s01);
                const uint32_t pl = ch / (4 * rpc), rr = (ch >> 2) - pl * rpc, p = g0 + pl, row = row0 + rr;
                const bool ok = c < nch && (c & 3u) == 0 && p < nx && row < rows;
                if (ok) {
                    const float yo = __uint_as_float(lds_ld32(Y + 256 * (i & 1) + 4 * (p * rpc + rr)));
                    gst_x1(a.y + (size_t)p * a.ystride + row, __float_as_uint(yo + tot));
                }
                if (__ballot(ok) != 0) ++ops;                     // counted only when some lane stores
            }
        }
    }
    WAIT_VM(0);
}

static size_t sbl_smem(bool q8, bool iq, uint32_t W, uint32_t slot, uint32_t nsb) {
    const size_t xs = ((q8 ? nsb * 8 * SBL_X8 : nsb * SBL_XS) + 1023u) & ~(size_t)1023;
    return (size_t)W * 2 * slot + xs + (size_t)W * ((q8 ? 4096 : 1024) + 256) + (iq ? 3072 : 0);
}

int launch_dot_sbl(int fmt, const DotArgs & a, bool fuse, hipStream_t s, const NormArgs * norm) {
    const bool iq = fmt == FMT_IQ2_XXS || fmt == FMT_IQ3_XXS;
    const bool q8 = fmt == FMT_Q8_0 || fmt == FMT_Q5_0 || iq;     // 32-weight blocks
    const bool q6 = fmt == FMT_Q6_K;
    if ((fmt != FMT_Q4_K && !q6 && !q8) || ((q8 || q6) && fuse) || a.nx != 1 || (a.cols & 255) || a.rows == 0)
        return FLH_ERR_UNSUPPORTED;
    const uint32_t nsb = a.cols >> 8, P = q8 ? 2 * nsb : nsb;
    const uint32_t B = fmt == FMT_Q4_K ? 144 : q6 ? 210 : fmt == FMT_Q8_0 ? 136 : fmt == FMT_Q5_0 ? 88
                                              : iq_block_bytes(fmt) / 2;
    // rows of more than 64 four-block halves (32-weight-block formats, more
    // than 8192 columns): two halves per lane, whose 4 chains of P terms fit
    // the wave's 4 KiB of fold terms up to 63 superblocks (16128 columns)
    const uint32_t H = q8 && P > 64 ? 2 : 1, PL = P / H;
    if (nsb < 1 || PL > 64 || (H == 2 && 4 * (8 * P + 16) > 4096)) return FLH_ERR_UNSUPPORTED;
    // chunks are whole rows moved in 16-byte pieces (IQ rows: nsb % 8 == 0)
    if ((P * B) & 15) return FLH_ERR_UNSUPPORTED;
    if ((uintptr_t)a.w & 15 || (a.estride & 15)) return FLH_ERR_UNSUPPORTED;
    if ((fuse || q8) && ((uintptr_t)a.x & 15)) return FLH_ERR_UNSUPPORTED;
    const Tune & t = tune();
    const uint32_t rpc = 64 / PL;
    const uint32_t ni = (rpc * P * B + 1023) / 1024, slot = ni * 1024;
    // Measured defaults (layer shapes, graph-replayed launches):
    //  * fused: 8 waves (the quantisation is shared by more waves), 4 of
    //    them requesting a chunk before the activation is ready; above 2^18
    //    superblocks the four-lanes-per-superblock kernel is faster and this
    //    launcher declines (fused, us, this kernel vs that one: 10240x4096
    //    7.62 vs 9.10, 14336x4096 9.14 vs 9.61, 16384x4096 9.91 vs 10.28,
    //    6144x8192 10.48 vs 10.61; 20480x4096 11.37 vs 11.11, gate/up
    //    28672x4096 14.74 vs 13.47, 12288x8192 16.09 vs 13.34);
    //  * unfused, <= 16 superblocks per row: 4 waves, 2 early (O 4096x4096
    //    5.37 -> 4.85 us, QKV 5.95 -> 5.49);
    //  * unfused, wider rows: 8 waves, 4 early (down 4096x14336 9.78 -> 9.63);
    //  * Q8_0: 4 waves, all early (4096x4096 6.98 -> 6.31 us, 14336x4096
    //    13.53 -> 13.27 against 8 waves);
    //  * Q5_0 and the IQ formats, more VALU work per byte: 8 waves, all
    //    early (14336x4096 Q5_0 15.2 -> 11.9 us, IQ2_XXS 16.6 -> 12.2,
    //    IQ3_XXS 18.3 -> 13.5 against 4 waves).
    // (NORM: against an RMSNORM launch of its own, at every size)
    if (fuse && !norm && !t.sbl_w && (uint64_t)a.rows * nsb > (1u << 18)) return FLH_ERR_UNSUPPORTED;
    //  * unfused Q4_K rows of more than 16 superblocks: above 2^18
    //    superblocks the four-lanes kernel streams them faster (us, this
    //    kernel vs that one: 8192x14336 15.68 vs 14.86; 4096x14336 9.41 vs
    //    9.64, 4096x8192 7.07 vs 7.20; 28672x4096, 16 per row, 13.31 vs 13.49)
    if (!fuse && fmt == FMT_Q4_K && nsb > 16 && !t.sbl_w && (uint64_t)a.rows * nsb > (1u << 18))
        return FLH_ERR_UNSUPPORTED;
    if (norm && (fmt != FMT_Q4_K || !fuse || ((uintptr_t)norm->x & 15) || ((uintptr_t)norm->wn & 15)))
        return FLH_ERR_UNSUPPORTED;
    // Q6_K: its 6-bit decode is VALU-heavy and a 12-14 KB chunk leaves room
    // for 4 waves only, so the four-lanes-per-superblock kernel stays faster
    // unless the matrix is large enough for the streaming rate to dominate
    // (measured: vocab 128256x4096 66.3 vs 68.6 us; 14336x4096 12.0 vs 10.8,
    // 4096x14336 13.9 vs 12.1, 4096x4096 5.8 either way)
    if (q6 && !t.sbl_w && (uint64_t)a.rows * nsb < (1u << 20)) return FLH_ERR_UNSUPPORTED;
    const uint32_t wdef = fuse || nsb > 16 || (q8 && fmt != FMT_Q8_0) ? 8 : 4;
    uint32_t W = t.sbl_w ? t.sbl_w : wdef;
    const uint32_t pre = t.sbl_pre == 0xFFu ? W : t.sbl_pre ? t.sbl_pre : q8 ? W : W / 2;
    // (NORM: its kernel's static LDS, the norm partials, comes on top; it
    // runs 8 or 4 waves)
    const size_t lim = lds_limit() - (norm ? std::max(static_lds((const void *)k_dot_sbl<FMT_Q4_K, true, 8, false, true>),
                                                      static_lds((const void *)k_dot_sbl<FMT_Q4_K, true, 4, false, true>))
                                           : 0);
    while (W > 4 && (sbl_smem(q8, iq, W, slot, nsb) > lim || (norm && W != 8 && W != 4))) W -= 2;
    const size_t smb = sbl_smem(q8, iq, W, slot, nsb);
    if (smb > lim || (W != 8 && W != 6 && W != 4)) return FLH_ERR_UNSUPPORTED;
    if (fuse && (nsb + W - 1) / W > 8) return FLH_ERR_UNSUPPORTED;
    // NORM: the items' fp32 x and norm weights share the second ring stage
    if (norm && ((W != 8 && W != 4) || (nsb + W - 1) / W > 4 || 8 * 1024 > slot)) return FLH_ERR_UNSUPPORTED;
    const uint32_t C = (a.rows + rpc - 1) / rpc;
    const uint32_t wpc = t.sbl_wpc ? t.sbl_wpc : 1;
    uint32_t G = (uint32_t)num_cus() * wpc;
    if (t.sbl_gmax && G > t.sbl_gmax) G = t.sbl_gmax;
    if (G > C) G = C;
    auto go = [&](auto kern) {
        if (int rc = lds_fits((const void *)kern, smb, "k_dot_sbl: LDS over the limit")) return rc;
        (void)hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smb);
        hipLaunchKernelGGL(kern, dim3(G), dim3(64 * W), smb, s, a, rpc, ni, slot, pre, MoeArgs{},
                           norm ? *norm : NormArgs{});
        return hip_check(hipGetLastError(), "k_dot_sbl launch");
    };
    auto unfused = [&](auto fmt_tag) {
        constexpr int F = decltype(fmt_tag)::value;
        if constexpr (F != FMT_Q4_K && F != FMT_Q6_K) {
            if (H == 2) {
                if (W == 8) return go(k_dot_sbl<F, false, 8, false, false, 2>);
                if (W == 6) return go(k_dot_sbl<F, false, 6, false, false, 2>);
                return go(k_dot_sbl<F, false, 4, false, false, 2>);
            }
        }
        if (W == 8) return go(k_dot_sbl<F, false, 8>);
        if (W == 6) return go(k_dot_sbl<F, false, 6>);
        return go(k_dot_sbl<F, false, 4>);
    };
    switch (fmt) {
        case FMT_Q6_K: return unfused(std::integral_constant<int, FMT_Q6_K>());
        case FMT_Q8_0: return unfused(std::integral_constant<int, FMT_Q8_0>());
        case FMT_Q5_0: return unfused(std::integral_constant<int, FMT_Q5_0>());
        case FMT_IQ2_XXS: return unfused(std::integral_constant<int, FMT_IQ2_XXS>());
        case FMT_IQ3_XXS: return unfused(std::integral_constant<int, FMT_IQ3_XXS>());
        default: break;
    }
    if (!fuse) return unfused(std::integral_constant<int, FMT_Q4_K>());
    if (norm) return W == 8 ? go(k_dot_sbl<FMT_Q4_K, true, 8, false, true>) : go(k_dot_sbl<FMT_Q4_K, true, 4, false, true>);
    if (W == 8) return go(k_dot_sbl<FMT_Q4_K, true, 8>);
    if (W == 6) return go(k_dot_sbl<FMT_Q4_K, true, 6>);
    return go(k_dot_sbl<FMT_Q4_K, true, 4>);
}

// Several activation columns (2..16) of a 32-weight-block format: one pass
// over the weights for up to 8 columns (capacity 2, 4 or 8; columns past nx
// read column 0 and store nothing), two passes for 9..16.  FLH_ERR_UNSUPPORTED (nothing launched)
// when a row spans more than 64 lanes (over 8192 columns), a chunk's rows
// would need more than 64 old-y words, or the LDS plan does not fit.
static int sbl_nx_go(int fmt, const DotArgs & a, hipStream_t s, bool dry);
int launch_dot_sbl_nx(int fmt, const DotArgs & a, hipStream_t s) { return sbl_nx_go(fmt, a, s, false); }

// dry: FLH_OK when the launch would go ahead, launching nothing
static int sbl_nx_go(int fmt, const DotArgs & a, hipStream_t s, bool dry) {
    const bool iq = fmt == FMT_IQ2_XXS || fmt == FMT_IQ3_XXS;
    if ((fmt != FMT_Q8_0 && fmt != FMT_Q5_0 && !iq) || a.nx < 2 || a.nx > 16 || (a.cols & 255) || a.rows == 0)
        return FLH_ERR_UNSUPPORTED;
    if (a.nx > 8) {
        // 9..16 columns: a pass of up to 8 and one of the rest (at least 2;
        // each column's result is its own, so the split changes no bits).
        // Nothing is launched unless both plans fit (the caller's fallback
        // must not add to y twice).
        DotArgs lo = a, hi = a;
        lo.nx = a.nx - 8 >= 2 ? 8 : a.nx - 2;
        hi.nx = a.nx - lo.nx;
        hi.x = a.x + (size_t)lo.nx * a.xstride;
        hi.y = a.y + (size_t)lo.nx * a.ystride;
        if (sbl_nx_go(fmt, lo, s, true) != FLH_OK || sbl_nx_go(fmt, hi, s, true) != FLH_OK)
            return FLH_ERR_UNSUPPORTED;
        if (dry) return FLH_OK;
        const int rc = sbl_nx_go(fmt, lo, s, false);
        return rc != FLH_OK ? rc : sbl_nx_go(fmt, hi, s, false);
    }
    const uint32_t nsb = a.cols >> 8, P = 2 * nsb;
    const uint32_t B = fmt == FMT_Q8_0 ? 136 : fmt == FMT_Q5_0 ? 88 : iq_block_bytes(fmt) / 2;
    if (P > 64 || ((P * B) & 15) || ((uintptr_t)a.w & 15) || (a.estride & 15) || ((uintptr_t)a.x & 3))
        return FLH_ERR_UNSUPPORTED;
    const uint32_t NX = a.nx <= 2 ? 2 : a.nx <= 4 ? 4 : 8;
    const uint32_t rpc = 64 / P;
    if (NX * rpc > 64) return FLH_ERR_UNSUPPORTED;
    const uint32_t ni = (rpc * P * B + 1023) / 1024, slot = ni * 1024;
    const Tune & t = tune();
    // plan: 8 waves with a 1-stage ring (refilled right after the decode)
    // and at least 2 columns parked at once, else 4 waves with 2 stages and
    // the most columns parked at once.  Measured at 14336x4096 (us, N = 2 /
    // 4 / 8): 8 waves x 1 stage Q8_0 14.0 / 18.5 / 27.6, Q5_0 15.4 / 18.4 /
    // 27.6, IQ2_XXS 13.5 / 16.1 / 23.2, IQ3_XXS 15.4 / 17.9 / 25.1; with 2
    // stages (8 waves where they fit, else 4) Q8_0 18.1 / 21.8 / 33.0, Q5_0
    // 15.3 / 21.3 / 37.0, IQ3_XXS 15.4 / 17.9 / 29.1 (two waves per SIMD hide
    // the per-column LDS round trips; one column parked at a time loses)
    auto smem = [&](uint32_t W, uint32_t d, uint32_t cg) {
        return (size_t)W * d * slot + sbl_nx_xq_bytes(NX, nsb) + sbl_nx_xd_bytes(NX, nsb) +
               (size_t)W * sbl_nx_tw(cg, rpc, P) + (iq ? 3072 : 0);
    };
    uint32_t W = 0, CG = 0, dep = 0;
    const uint32_t plans[3][2] = {{8, 1}, {4, 2}, {8, 2}};   // the last: forced 8 waves x 2 stages
    for (const auto & pl : plans) {
        const uint32_t w = pl[0], d = pl[1];
        if ((t.sbl_w && t.sbl_w != w) || (t.sbl_nx_dep && t.sbl_nx_dep != d)) continue;
        for (uint32_t cg = NX < 4 ? NX : 4; cg >= (w == 8 && !t.sbl_w ? 2u : 1u) && !W; cg >>= 1)
            if (smem(w, d, cg) <= lds_limit()) { W = w; CG = cg; dep = d; }
        if (W) break;
    }
    if (!W) return FLH_ERR_UNSUPPORTED;
    if (dry) return FLH_OK;
    const size_t smb = smem(W, dep, CG);
    const uint32_t pre = t.sbl_pre == 0xFFu ? W : t.sbl_pre ? t.sbl_pre : W;
    const uint32_t C = (a.rows + rpc - 1) / rpc;
    uint32_t G = (uint32_t)num_cus() * (t.sbl_wpc ? t.sbl_wpc : 1);
    if (t.sbl_gmax && G > t.sbl_gmax) G = t.sbl_gmax;
    if (G > C) G = C;
    auto go = [&](auto kern) {
        if (int rc = lds_fits((const void *)kern, smb, "k_dot_sbl: LDS over the limit")) return rc;
        (void)hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smb);
        hipLaunchKernelGGL(kern, dim3(G), dim3(64 * W), smb, s, a, rpc, ni, slot, pre, NX, dep);
        return hip_check(hipGetLastError(), "k_dot_sbl_nx launch");
    };
    auto by_cg = [&](auto fmt_tag, auto w_tag) {
        constexpr int F = decltype(fmt_tag)::value, WW = decltype(w_tag)::value;
        if (CG == 4) return go(k_dot_sbl_nx<F, WW, 4>);
        if (CG == 2) return go(k_dot_sbl_nx<F, WW, 2>);
        return go(k_dot_sbl_nx<F, WW, 1>);
    };
    auto by_w = [&](auto fmt_tag) {
        if (W == 8) return by_cg(fmt_tag, std::integral_constant<int, 8>());
        return by_cg(fmt_tag, std::integral_constant<int, 4>());
    };
    switch (fmt) {
        case FMT_Q8_0: return by_w(std::integral_constant<int, FMT_Q8_0>());
        case FMT_Q5_0: return by_w(std::integral_constant<int, FMT_Q5_0>());
        case FMT_IQ2_XXS: return by_w(std::integral_constant<int, FMT_IQ2_XXS>());
        default: return by_w(std::integral_constant<int, FMT_IQ3_XXS>());
    }
}

// Routed expert dots, one workgroup row per (token, slot) pair, the dense
// launch's workgroups shared evenly by the pairs: Q4_K for one token (more
// tokens share experts on the grouped kernels), the 32-weight-block formats
// for any batch (no grouping; ntok * top_k <= 256).  Measured at Mixtral
// shapes (8 experts, top 2, batch 1) against the four-lanes-per-superblock
// grouped kernel: gate/up 2 x 28672x4096 with ROUTER_SEL fused 26.5 -> 25.0
// us, down 2 x 4096x14336 16.2 -> 15.8 us.  The routed gate/up still trails a
// dense 57344x4096 launch (22.3 us) by the routing itself: no weight request
// can leave before the logits are loaded and ranked.
int launch_moe_sbl(int fmt, const MoeArgs & m, hipStream_t s) {
    const bool iq = fmt == FMT_IQ2_XXS || fmt == FMT_IQ3_XXS;
    const bool q8 = fmt == FMT_Q8_0 || fmt == FMT_Q5_0 || iq;     // 32-weight blocks
    const uint32_t pairs = m.ntok * m.top_k;
    if ((fmt != FMT_Q4_K && !q8) || (fmt == FMT_Q4_K && m.ntok != 1) || pairs == 0 || pairs > 256 ||
        (m.cols & 255) || m.rows == 0)
        return FLH_ERR_UNSUPPORTED;
    const uint32_t nsb = m.cols >> 8, P = q8 ? 2 * nsb : nsb;
    const uint32_t B = fmt == FMT_Q4_K ? 144 : fmt == FMT_Q8_0 ? 136 : fmt == FMT_Q5_0 ? 88 : iq_block_bytes(fmt) / 2;
    // two four-block halves per lane above 64 (as launch_dot_sbl)
    const uint32_t H = q8 && P > 64 ? 2 : 1, PL = P / H;
    if (nsb < 1 || PL > 64 || (H == 2 && 4 * (8 * P + 16) > 4096) || ((P * B) & 15)) return FLH_ERR_UNSUPPORTED;
    if ((uintptr_t)m.w & 15 || (m.estride & 15)) return FLH_ERR_UNSUPPORTED;
    if (q8 && (((uintptr_t)m.x & 15) || (m.xstride & 3))) return FLH_ERR_UNSUPPORTED;
    const Tune & t = tune();
    const uint32_t rpc = 64 / PL;
    const uint32_t ni = (rpc * P * B + 1023) / 1024, slot = ni * 1024;
    uint32_t W = t.sbl_w ? t.sbl_w : nsb > 16 || (q8 && fmt != FMT_Q8_0) ? 8 : 4;
    const uint32_t pre = t.sbl_pre == 0xFFu ? W : t.sbl_pre ? t.sbl_pre : q8 ? W : W / 2;
    const size_t lim = lds_limit() - 1088;                        // the routed ids (static LDS)
    while (W > 4 && sbl_smem(q8, iq, W, slot, nsb) > lim) W -= 2;
    const size_t smb = sbl_smem(q8, iq, W, slot, nsb);
    if (smb > lim || (W != 8 && W != 6 && W != 4)) return FLH_ERR_UNSUPPORTED;
    const uint32_t C = (m.rows + rpc - 1) / rpc;
    const uint32_t wpc = t.sbl_wpc ? t.sbl_wpc : 1;
    uint32_t G = (uint32_t)num_cus() * wpc;
    if (t.sbl_gmax && G > t.sbl_gmax) G = t.sbl_gmax;
    uint32_t gx = (G + pairs - 1) / pairs;
    if (gx > C) gx = C;
    DotArgs a{};
    a.w = m.w;
    a.rows = m.rows;
    a.cols = m.cols;
    a.nx = 1;
    auto go = [&](auto kern) {
        if (int rc = lds_fits((const void *)kern, smb, "k_dot_sbl: LDS over the limit")) return rc;
        (void)hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smb);
        hipLaunchKernelGGL(kern, dim3(gx, pairs), dim3(64 * W), smb, s, a, rpc, ni, slot, pre, m, NormArgs{});
        return hip_check(hipGetLastError(), "k_dot_sbl (moe) launch");
    };
    auto routed = [&](auto fmt_tag) {
        constexpr int F = decltype(fmt_tag)::value;
        if constexpr (F != FMT_Q4_K) {
            if (H == 2) {
                if (W == 8) return go(k_dot_sbl<F, false, 8, true, false, 2>);
                if (W == 6) return go(k_dot_sbl<F, false, 6, true, false, 2>);
                return go(k_dot_sbl<F, false, 4, true, false, 2>);
            }
        }
        if (W == 8) return go(k_dot_sbl<F, false, 8, true>);
        if (W == 6) return go(k_dot_sbl<F, false, 6, true>);
        return go(k_dot_sbl<F, false, 4, true>);
    };
    switch (fmt) {
        case FMT_Q8_0: return routed(std::integral_constant<int, FMT_Q8_0>());
        case FMT_Q5_0: return routed(std::integral_constant<int, FMT_Q5_0>());
        case FMT_IQ2_XXS: return routed(std::integral_constant<int, FMT_IQ2_XXS>());
        case FMT_IQ3_XXS: return routed(std::integral_constant<int, FMT_IQ3_XXS>());
        default: return routed(std::integral_constant<int, FMT_Q4_K>());
    }
}

}  // namespace flh
