// flh_kstream.h -- device building blocks of the LDS-staged int8 x q8_K
// row-dot (Q4_K / Q6_K), shared by the single-matrix kernels
// (flh_dot_kstream.hip) and their fused / grouped variants.
//
// Weight bytes go HBM -> LDS with direct-to-LDS dwordx4 loads
// (global_load_lds_dwordx4) in one fully coalesced pass.  Work unit: a CHUNK
// of 16 consecutive superblocks of the row-major matrix (a chunk may straddle
// rows).  Lane (slot s = lane/4, part c = lane%4) of a wave computes the exact
// integer partials of superblock s, quarter c; the partials are reduced across
// the quad with DPP and parked in LDS as (row, column, superblock) terms; a
// fold pass then applies the reference's float order per (row, column,
// accumulator), so results are bitwise equal to fl_dot_i8k_q4_K /
// fl_dot_i8k_q6_K (src/runtime/quants.h:538-594).
//
// The activation (q8_K appendix, or fp32 x quantised in place of ACT_Q8) is
// re-laid in LDS as 80-byte per-lane records (64 int8 + 4 int32 block sums).
#pragma once
#include "flh_common.h"
#include "flh_internal.h"

namespace flh {

// Development timing probe (compiled only with -DFLH_TRACE): per workgroup of
// the streaming kernel, s_memrealtime stamps at entry (0), after activation
// staging (1), at the first landed chunk (2), after the last chunk (3), at
// exit (4), when the activation loads have landed (5), before the staging
// barrier (6), at the second landed chunk (7), after wave 0's last chunk of
// the last batch (12), after the last fold (8), after the fused quantisation
// (11); slot 15 holds the hardware ids (XCC_ID << 32 | HW_ID).
#ifdef FLH_TRACE
__device__ uint64_t g_ks_trace[8192 * 16];
#define KS_STAMP(k) do { if (threadIdx.x == 0 && blockIdx.x < 8192) { \
    g_ks_trace[(size_t)blockIdx.x * 16 + (k)] = __builtin_amdgcn_s_memrealtime(); \
    if ((k) == 0) g_ks_trace[(size_t)blockIdx.x * 16 + 15] = \
        ((uint64_t)__builtin_amdgcn_s_getreg((20) | (0 << 6) | (3 << 11)) << 32) | \
        (uint64_t)__builtin_amdgcn_s_getreg((4) | (0 << 6) | (31 << 11)); } } while (0)
#else
#define KS_STAMP(k) do { } while (0)
#endif

#define GPTR(p) ((const void __attribute__((address_space(1))) *)(p))
#define LPTR(p) ((void __attribute__((address_space(3))) *)(p))

// s_waitcnt vmcnt(n) only (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14])
#define WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (0x7 << 4) | (0xF << 8) | (((n) >> 4) << 14))
#define WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)

// Cache-policy bits of the weight-streaming DMA (2 = nontemporal: the weights
// are read once per launch and should not displace the activation in L2).
#ifndef FLH_KS_AUX
#define FLH_KS_AUX 2
#endif

// Workgroup barrier for LDS data only: waits for this wave's LDS operations,
// not for its outstanding global loads, so the direct-to-LDS weight DMAs stay
// in flight across it (each wave waits for its own stages explicitly).
// __syncthreads() would also wait for every outstanding global load.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

typedef uint32_t u32x4a __attribute__((ext_vector_type(4)));

// LDS offset of a pointer into __shared__ memory
__device__ __forceinline__ uint32_t lds_off(const void * p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// LDS accesses hidden from the compiler's wait-count pass.  A plain LDS access
// issued while direct-to-LDS DMAs are in flight makes the compiler wait for
// every outstanding global load (it cannot tell the LDS regions apart); these
// wait only for the loads that produce their register operands.  Reads wait
// for their own completion inside the asm.
__device__ __forceinline__ void lds_st128(void * p, u32x4a v) {
    asm volatile("ds_write_b128 %0, %1" :: "v"(lds_off(p)), "v"(v));
}
__device__ __forceinline__ void lds_st32(void * p, uint32_t v) {
    asm volatile("ds_write_b32 %0, %1" :: "v"(lds_off(p)), "v"(v));
}
__device__ __forceinline__ void lds_max32(void * p, uint32_t v) {
    asm volatile("ds_max_u32 %0, %1" :: "v"(lds_off(p)), "v"(v));
}
__device__ __forceinline__ uint32_t lds_ld32(const void * p) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_off(p)) : "memory");
    return v;
}
// five consecutive 16-byte words (one 80-byte activation record)
__device__ __forceinline__ void lds_ld_rec(const void * p, u32x4a (&v)[5]) {
    asm volatile("ds_read_b128 %0, %5\n\tds_read_b128 %1, %5 offset:16\n\tds_read_b128 %2, %5 offset:32\n\t"
                 "ds_read_b128 %3, %5 offset:48\n\tds_read_b128 %4, %5 offset:64\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]) : "v"(lds_off(p)) : "memory");
}

// Activation loads hidden from the compiler's wait-count pass.  A register
// load followed by direct-to-LDS DMAs makes the compiler wait for every DMA
// (vmcnt(0)) before the loaded value is used, i.e. for the first weight
// chunks as well.  These loads are issued before the weight prologue; the
// caller then waits with ks_wait_behind for exactly the DMAs issued after them
// and passes the values through xfence() before use (the fence orders the uses
// after that wait; each value stays in the register the load wrote).
__device__ __forceinline__ u32x4a gld_x4(const void * p) {
    u32x4a r;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return r;
}
__device__ __forceinline__ uint32_t gld_x1(const void * p) {
    uint32_t r;
    asm volatile("global_load_dword %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return r;
}
__device__ __forceinline__ uint32_t gld_xs16(const void * p) {      // sign-extended int16
    uint32_t r;
    asm volatile("global_load_sshort %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return r;
}
__device__ __forceinline__ uint32_t gld_xu16(const void * p) {
    uint32_t r;
    asm volatile("global_load_ushort %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return r;
}
__device__ __forceinline__ void xfence(u32x4a & v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void xfence(uint32_t & v) { asm volatile("" : "+v"(v)); }

template <int FMT> struct KS;
template <> struct KS<FMT_Q4_K> {
    static constexpr uint32_t BLK = 144;
    static constexpr uint32_t WIN = 2304;            // LDS bytes per chunk stage
    static constexpr int NI = 3;                     // DMA instructions per chunk
};
template <> struct KS<FMT_Q6_K> {
    static constexpr uint32_t BLK = 210;
    static constexpr uint32_t WIN = 4096;            // 3360 B + realignment slack
    static constexpr int NI = 4;
};
// Q8_0: a "superblock" is a unit of 8 blocks (256 weights, 272 bytes, 16-byte
// aligned in a row-major matrix whose rows hold a multiple of 256 weights)
template <> struct KS<FMT_Q8_0> {
    static constexpr uint32_t BLK = 272;
    static constexpr uint32_t WIN = 4352;            // 16 units: 4 x 1024 B + 256 B
    static constexpr int NI = 5;
};
// fold terms per superblock (Q8_0 folds per 32-weight block)
template <int FMT> __host__ __device__ constexpr uint32_t ks_tps() { return FMT == FMT_Q8_0 ? 8 : 1; }

constexpr uint32_t XREC = 80;                        // bytes per (sb, part) activation record

// LDS of the records of nx columns of nsb superblocks, and of the fold terms
// of nr rows
template <int FMT>
__host__ __device__ inline size_t ks_xrec_bytes(uint32_t nx, uint32_t nsb) {
    return (size_t)nx * nsb * 4 * XREC + (size_t)nx * nsb * 4 * ks_tps<FMT>();
}
template <int FMT>
__host__ __device__ inline size_t ks_term_bytes(uint32_t nr, uint32_t nx, uint32_t nsb) {
    return ((size_t)nr * nx * nsb * 4 * (FMT == FMT_Q4_K ? 2 : 1) + (size_t)nr * nsb * 4) * ks_tps<FMT>();
}
template <int FMT>
__host__ __device__ inline size_t ks_smem_bytes(uint32_t nr, uint32_t nx, uint32_t nsb, int D, int KW = 4) {
    return (size_t)KW * D * KS<FMT>::WIN + ks_xrec_bytes<FMT>(nx, nsb) + ks_term_bytes<FMT>(nr, nx, nsb) + 256;
}

// Wait until at most `behind` chunks' DMAs (NI loads each) are outstanding;
// behind < D is wave-uniform.
template <int NI, int D>
__device__ __forceinline__ void ks_wait_behind(uint32_t behind) {
    if (D > 4 && behind >= 4) { WAIT_VM(NI * (D > 4 ? 4 : 0)); return; }
    if (D > 3 && behind >= 3) { WAIT_VM(NI * (D > 3 ? 3 : 0)); return; }
    if (D > 2 && behind >= 2) { WAIT_VM(NI * (D > 2 ? 2 : 0)); return; }
    if (D > 1 && behind >= 1) { WAIT_VM(NI); return; }
    WAIT_VM(0);
}

// Issue the DMA of chunk `ch` (batch-local) into a stage.  Lanes past the
// chunk's valid bytes re-read the last valid 16 bytes (never out of bounds).
template <int FMT>
__device__ __forceinline__ void ks_issue(const uint8_t * wb, uint32_t ch, uint32_t nsb_batch,
                                         uint8_t * stage, uint32_t lane) {
    constexpr uint32_t B = KS<FMT>::BLK;
    const uint32_t f0 = ch * 16;
    const uint32_t nact = nsb_batch - f0 < 16 ? nsb_batch - f0 : 16;
    if constexpr (FMT == FMT_Q4_K) {
        const uint8_t * g = wb + (size_t)f0 * B;
        const uint32_t last16 = nact * B - 16, last4 = nact * B - 4;
        const uint32_t o0 = 16 * lane, o1 = 1024 + 16 * lane, o2 = 2048 + 4 * lane;
        __builtin_amdgcn_global_load_lds(GPTR(g + (o0 <= last16 ? o0 : last16)), LPTR(stage), 16, 0, FLH_KS_AUX);
        __builtin_amdgcn_global_load_lds(GPTR(g + (o1 <= last16 ? o1 : last16)), LPTR(stage + 1024), 16, 0, FLH_KS_AUX);
        __builtin_amdgcn_global_load_lds(GPTR(g + (o2 <= last4 ? o2 : last4)), LPTR(stage + 2048), 4, 0, FLH_KS_AUX);
    } else if constexpr (FMT == FMT_Q8_0) {
        const uint8_t * g = wb + (size_t)f0 * B;
        const uint32_t last16 = nact * B - 16, last4 = nact * B - 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t o = 1024 * i + 16 * lane;
            __builtin_amdgcn_global_load_lds(GPTR(g + (o <= last16 ? o : last16)), LPTR(stage + 1024 * i), 16, 0, FLH_KS_AUX);
        }
        const uint32_t o4 = 4096 + 4 * lane;
        __builtin_amdgcn_global_load_lds(GPTR(g + (o4 <= last4 ? o4 : last4)), LPTR(stage + 4096), 4, 0, FLH_KS_AUX);
    } else {
        const uintptr_t gs = (uintptr_t)(wb + (size_t)f0 * B);
        const uint8_t * g = (const uint8_t *)(gs & ~(uintptr_t)15);
        const uint32_t last16 = (uint32_t)((gs + nact * B - 1) - (uintptr_t)g) & ~15u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t o = 1024 * i + 16 * lane;
            __builtin_amdgcn_global_load_lds(GPTR(g + (o <= last16 ? o : last16)), LPTR(stage + 1024 * i), 16, 0, FLH_KS_AUX);
        }
    }
}

// 16 bytes at an even LDS byte offset (realigned from 5 aligned dwords)
__device__ __forceinline__ void lds16_u2(const uint8_t * base, uint32_t off, uint32_t (&o)[4]) {
    const uint32_t * p = (const uint32_t *)(base + (off & ~3u));
    const uint32_t sh = off & 3u;
    uint32_t d[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) d[i] = p[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = alignb(d[i + 1], d[i], sh);
}

// Position of x element e (0..255 of a superblock) in the per-lane records:
// which part c, which 16-byte slot k, byte offset inside the slot.
template <int FMT>
__device__ __forceinline__ void xrec_pos(uint32_t e, uint32_t & cc, uint32_t & k, uint32_t & t) {
    if constexpr (FMT == FMT_Q4_K) {      // part c owns groups {g0, g0+1, g0+4, g0+5}, half c&1
        const uint32_t g = e >> 5, h = (e >> 4) & 1;
        cc = 2 * ((g & 3) >> 1) + h;
        k = (g & 1) + 2 * (g >> 2);
        t = e & 15;
    } else {                              // part c = (half hh, 16-run bb) owns groups 0..3
        const uint32_t hh = e >> 7, g = (e >> 5) & 3, bb = (e >> 4) & 1;
        cc = 2 * hh + bb;
        k = g;
        t = e & 15;
    }
}

// Columns of one kstream pass: x_p / y_p base pointers (p < nx <= NX).
template <int NX>
struct KsCols {
    const float * x[NX];
    float * y[NX];
};
// runtime column select without dynamic register indexing
// (each candidate passes through an empty asm so that the compiler cannot fold
// the select chain back into an indexed access of a stack array, which a
// lane-varying p would turn into scratch memory)
template <int NX, typename T>
__device__ __forceinline__ T col_pick(T const (&v)[NX], uint32_t p) {
    uint64_t r = (uint64_t)v[0];
#pragma unroll
    for (int i = 1; i < NX; ++i) {
        uint64_t vi = (uint64_t)v[i];
        asm volatile("" : "+v"(vi));
        r = p == (uint32_t)i ? vi : r;
    }
    return (T)r;
}

// ---------------------------------------------------------------- ACT_Q8 --
// One wave quantises one 256-element chunk: lane i holds elements 4i..4i+3
// in v.  Writes the chunk's q8_1 blocks (8-lane groups) and its q8_K block
// with the bytes of fl_quantize_q8_1_block / fl_quantize_q8_K_block
// (src/runtime/quants.h:360-402): amax is a max (order free), d = amax/127
// and id = 127/amax are correctly rounded IEEE divisions, q = roundf(x*id)
// clamped to +-127, sums are exact integers, halves are RNE.
// q = roundf(y) clamped to [-127, 127] (the reference quantizers' step), as
// an integer: for every float |y| <= 128.5, trunc(y + copysign(0.5 - 2^-25, y))
// equals roundf(y) (checked exhaustively over all such floats; a CPU test
// pins the cases near every integer and half-integer), v_cvt_i32_f32
// truncates, and larger |y| saturate to +-127 either way.
__device__ __forceinline__ int q8_round(float y) {
    const float t = y + __builtin_copysignf(0.49999997f, y);
    const int q = (int)t;
    return q < -127 ? -127 : q > 127 ? 127 : q;
}
// four values quantised with scale id, packed little-endian as int8
__device__ __forceinline__ uint32_t quant4(const float (&v)[4], float id) {
    uint32_t packed = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) packed |= ((uint32_t)q8_round(v[j] * id) & 0xFFu) << (8 * j);
    return packed;
}
// max |v_j| from 0 (NaN never wins, as in the reference's "if (a > amax)")
__device__ __forceinline__ float absmax4(const float (&v)[4]) {
    return fmaxf(fmaxf(fmaxf(fmaxf(0.f, fabsf(v[0])), fabsf(v[1])), fabsf(v[2])), fabsf(v[3]));
}
__device__ __forceinline__ void act_q8_lanes(const float (&v)[4], uint32_t lane, uint32_t chunk,
                                             uint8_t * q81, uint8_t * q8k, uint32_t cols) {
    const uint32_t am = __float_as_uint(absmax4(v));
    // q8_1: block of 32 = 8 lanes
    {
        const uint32_t blk = chunk * 8 + (lane >> 3);
        const float amax = __uint_as_float(umax8(am));
        const float d = amax / 127.f;
        const float id = amax > 0.f ? 127.f / amax : 0.f;
        const uint32_t pk = quant4(v, id);
        const int sum = sum8i(dot4((int)pk, 0x01010101, 0));
        if ((blk + 1) * 32 <= cols) {
            uint8_t * o = q81 + (size_t)blk * 36;
            *(uint32_t *)(o + 4 + 4 * (lane & 7)) = pk;
            if ((lane & 7) == 0) *(uint32_t *)o = f2h(d) | (f2h(d * (float)sum) << 16);
        }
    }
    // q8_K: whole chunk
    if ((chunk + 1) * 256 <= cols) {
        const float amax = __uint_as_float(umax64(am));
        const float d = amax / 127.f;
        const float id = amax > 0.f ? 127.f / amax : 0.f;
        const uint32_t pk = quant4(v, id);
        const int s = sum4i(dot4((int)pk, 0x01010101, 0));
        uint8_t * o = q8k + (size_t)chunk * 292;
        *(uint32_t *)(o + 36 + 4 * lane) = pk;
        if ((lane & 3) == 0) *(int16_t *)(o + 4 + 2 * (lane >> 2)) = (int16_t)s;
        if (lane == 0) *(float *)o = d;
    }
}

// ACT_Q8 fused into the dot: quantise the fp32 columns into the records.
// Wave w takes superblocks (items i = p * nsb + sb) w, w + KW, ..., up to four
// at a time with their loads in flight together; lane l holds elements
// 4l..4l+3 of an item, so each load instruction reads one contiguous 1 KiB
// (every workgroup reads the whole column: a lane-strided pattern asked L2
// for four times the lines and made this prologue ~1 us slower).  The
// superblock's absmax is a wave max (order free); the lane's four quantised
// bytes form one dword of a record and a quad sum gives its 16-element block
// sum.  Workgroup app_g of app_G also writes both appendices of the items i
// with i % app_G == app_g (every item by exactly one workgroup, so no single
// workgroup carries all the stores) with k_act_q8's lane code,
// so the bytes in memory equal ACT_Q8's.  after_loads() runs once, right after
// the first activation loads are issued (the caller issues its weight
// prologue there, behind the older activation loads).
//
// NORM (one column, at most 8 items per wave, KW dividing 16): the items come
// from nm.x with their norm weights, the column is first normalised exactly
// as k_rmsnorm_act_q8_reg does it (that kernel's thread (v, l) sums elements
// 4l..4l+3 of superblocks v, v + 16, ... in turn; superblock s sits in wave
// s % KW here, which holds the partials of v = wave + KW q in the same
// order), y = (x * s) * wn is quantised, and the workgroup that writes a
// superblock's appendices also stores its y into C.x.
template <int FMT, int NX, int NI, int D, int KW = 4, bool NORM = false, typename F>
__device__ __forceinline__ void ks_x_fuse(const KsCols<NX> & C, uint32_t nx, uint32_t nsb, uint32_t cols,
                                          uint8_t * xr, float * xd, uint32_t app_g, uint32_t app_G,
                                          F && after_loads, const NormArgs & nm = NormArgs{}) {
    static_assert(!NORM || (NX == 1 && (KW == 4 || KW == 8)), "RMSNORM: one column, 16 % KW == 0");
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nitem = nx * nsb;
    // record slot of this lane's four elements (the same in every superblock)
    uint32_t cc, kk, t;
    xrec_pos<FMT>(4 * lane, cc, kk, t);
    const uint32_t magic = div_magic(nsb);                        // i / nsb, i < 2^16
    // Quantise items base + KW * j + wave (j < 4) from v: four superblock
    // absmaxes (wave max of the non-negative float bits; the lane max starts
    // at 0, so NaN never wins, as the reference's "if (a > amax)"), one
    // division sequence for the four scales (lanes 0..3), records and scales
    // to LDS, and this workgroup's share of the appendices.
    auto quant_group = [&](uint32_t base, const float (&v)[4][4]) {
        uint32_t am[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (base + KW * j + wave < nitem) am[j] = umax64(__float_as_uint(absmax4(v[j])));
        const float al = __uint_as_float(lane == 0 ? am[0] : lane == 1 ? am[1] : lane == 2 ? am[2] : am[3]);
        const float dl = al / 127.f;
        const float idl = al > 0.f ? 127.f / al : 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t i = base + KW * j + wave;
            if (i >= nitem) break;                                       // wave-uniform
            const uint32_t p = div_small(i, magic), sb = i - p * nsb;
            const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dl), j));
            const float id = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(idl), j));
            const uint32_t pk = quant4(v[j], id);
            const int sum = sum4i(dot4((int)pk, 0x01010101, 0));        // 16-element block sum
            uint8_t * rec = xr + (((size_t)p * nsb + sb) * 4 + cc) * XREC;
            lds_st32(rec + 16 * kk + t, pk);
            if ((lane & 3) == 0) lds_st32(rec + 64 + 4 * kk, (uint32_t)(FMT == FMT_Q4_K ? sum : 32 * sum));
            if (lane == 0) lds_st32(&xd[p * nsb + sb], __float_as_uint(d));
            if (i % app_G == app_g) {
                uint8_t * xc = (uint8_t *)col_pick<NX>(C.x, p);
                if constexpr (NORM)
                    *(float4 *)((float *)xc + 256 * sb + 4 * lane) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
                act_q8_lanes(v[j], lane, sb, xc + xq_off(cols), xc + xqk_off(cols), cols);
            }
        }
    };
    auto vload = [&](uint32_t i) -> const float * {
        if constexpr (NORM) return nm.x + 256 * i + 4 * lane;
        const uint32_t p = div_small(i, magic);
        return col_pick<NX>(C.x, p) + 256 * (i - p * nsb) + 4 * lane;
    };
    if (nitem <= 8 * KW) {
        // every item of this wave (at most 8) is loaded before the weight
        // prologue, and only these loads are waited for
        u32x4a r[8], rw[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (KW * j + wave < nitem) {
                r[j] = gld_x4(vload(KW * j + wave));
                if constexpr (NORM) rw[j] = gld_x4(nm.wn + 256 * (KW * j + wave) + 4 * lane);
            }
        ks_wait_behind<NI, D + 1>(after_loads());
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            xfence(r[j]);
            if constexpr (NORM) xfence(rw[j]);
        }
        if constexpr (NORM) {
            __shared__ __attribute__((aligned(16))) float nparts[16];
            constexpr uint32_t NQ = 16 / KW;
            float ss[NQ];
#pragma unroll
            for (uint32_t q = 0; q < NQ; ++q) ss[q] = 0.f;
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j) {
                if (KW * j + wave < nitem) {
                    const float x0 = __uint_as_float(r[j].x), x1 = __uint_as_float(r[j].y);
                    const float x2 = __uint_as_float(r[j].z), x3 = __uint_as_float(r[j].w);
                    float & t = ss[j % NQ];
                    t += x0 * x0;
                    t += x1 * x1;
                    t += x2 * x2;
                    t += x3 * x3;
                }
            }
#pragma unroll
            for (uint32_t q = 0; q < NQ; ++q) {
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) ss[q] += xor_lane(ss[q], o, lane);
                if (lane == 0) lds_st32(&nparts[wave + KW * q], __float_as_uint(ss[q]));
            }
            lds_barrier();
            u32x4a p0, p1, p2, p3;                                // the 16 totals in one LDS round trip
            asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:16\n\tds_read_b128 %2, %4 offset:32\n\t"
                         "ds_read_b128 %3, %4 offset:48\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(p0), "=&v"(p1), "=&v"(p2), "=&v"(p3) : "v"(lds_off(nparts)) : "memory");
            const uint32_t pv[16] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w,
                                     p2.x, p2.y, p2.z, p2.w, p3.x, p3.y, p3.z, p3.w};
            float tn = 0.f;
#pragma unroll
            for (int v = 0; v < 16; ++v) tn += __uint_as_float(pv[v]);
            const float sn = 1.0f / sqrtf(tn / (float)cols + nm.eps);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                r[j].x = __float_as_uint(__uint_as_float(r[j].x) * sn * __uint_as_float(rw[j].x));
                r[j].y = __float_as_uint(__uint_as_float(r[j].y) * sn * __uint_as_float(rw[j].y));
                r[j].z = __float_as_uint(__uint_as_float(r[j].z) * sn * __uint_as_float(rw[j].z));
                r[j].w = __float_as_uint(__uint_as_float(r[j].w) * sn * __uint_as_float(rw[j].w));
            }
        }
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            if (4 * KW * g >= nitem) break;
            float v[4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[j][0] = __uint_as_float(r[4 * g + j].x); v[j][1] = __uint_as_float(r[4 * g + j].y);
                v[j][2] = __uint_as_float(r[4 * g + j].z); v[j][3] = __uint_as_float(r[4 * g + j].w);
            }
            quant_group(4 * KW * g, v);
        }
    } else {
        bool issued = false;
        for (uint32_t base = 0; base < nitem; base += 4 * KW) {
            u32x4a r[4] = {};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t i = base + KW * j + wave;                 // wave-uniform
                if (i < nitem) r[j] = gld_x4(vload(i));
            }
            if (!issued) {
                after_loads();
                issued = true;
            }
            WAIT_VM(0);
            float v[4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xfence(r[j]);
                v[j][0] = __uint_as_float(r[j].x); v[j][1] = __uint_as_float(r[j].y);
                v[j][2] = __uint_as_float(r[j].z); v[j][3] = __uint_as_float(r[j].w);
            }
            quant_group(base, v);
        }
        if (!issued) after_loads();
    }
    KS_STAMP(11);
    // columns p >= nx of the template width read zero records
    for (uint32_t i = tid; i < (NX - nx) * nsb * 4 * (XREC / 4); i += 64 * KW)
        ((uint32_t *)(xr + (size_t)nx * nsb * 4 * XREC))[i] = 0u;
    for (uint32_t i = tid; i < (NX - nx) * nsb; i += 64 * KW) xd[nx * nsb + i] = 0.f;
    KS_STAMP(6);
}

// Base of superblock sb's activation in column x: its q8_K block (K formats)
// or its 8 q8_1 blocks (Q8_0).
template <int FMT>
__device__ __forceinline__ const uint8_t * ks_xsb(const uint8_t * x, uint32_t cols, uint32_t sb) {
    return FMT == FMT_Q8_0 ? x + xq_off(cols) + (size_t)sb * 288 : x + xqk_off(cols) + (size_t)sb * 292;
}

// Records from the appendices written by ACT_Q8.  after_loads() as above.
// Loads of record (sb, part cc) of a column from its appendix at xb (the
// superblock's base: q8_K for the K formats; for Q8_0, the unit's 8 q8_1
// blocks), hidden from the compiler (gld_x*): v = the record's 64 int8, bs =
// its raw block sums (Q4_K / Q6_K: int16; Q8_0: the two q8_1 halves d), dk =
// the q8_K f32 d bits.
template <int FMT>
__device__ __forceinline__ void ks_xrec_issue(const uint8_t * xb, uint32_t cc, u32x4a (&v)[4], uint32_t (&bs)[4],
                                              uint32_t & dk) {
    if constexpr (FMT == FMT_Q8_0) {
        const uint8_t * b0 = xb + 72 * cc;
        v[0] = gld_x4(b0 + 4);
        v[1] = gld_x4(b0 + 20);
        v[2] = gld_x4(b0 + 40);
        v[3] = gld_x4(b0 + 56);
        bs[0] = gld_xu16(b0);
        bs[1] = gld_xu16(b0 + 36);
        bs[2] = bs[3] = 0;
        dk = 0;
    } else if constexpr (FMT == FMT_Q4_K) {
        const uint32_t g0 = 2 * (cc >> 1), h = cc & 1;
        const uint32_t gs[4] = {g0, g0 + 1, g0 + 4, g0 + 5};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[k] = gld_x4(xb + 36 + 32 * gs[k] + 16 * h);
            bs[k] = gld_xs16(xb + 4 + 2 * (2 * gs[k] + h));
        }
        dk = gld_x1(xb);
    } else {
        const uint32_t hh = cc >> 1, bb = cc & 1;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            v[g] = gld_x4(xb + 36 + 128 * hh + 32 * g + 16 * bb);
            bs[g] = gld_xs16(xb + 4 + 2 * (8 * hh + 2 * g + bb));
        }
        dk = gld_x1(xb);
    }
}

template <int FMT, int NX, int NI, int D, typename F>
__device__ __forceinline__ void ks_x_app(const KsCols<NX> & C, uint32_t nx, uint32_t nsb, uint32_t cols,
                                         uint8_t * xr, float * xd, F && after_loads) {
    const uint32_t tid = threadIdx.x;
    if (NX * nsb * 4 <= 256) {
        // one record per thread: load, run after_loads (the weight prologue),
        // wait for the record loads alone, then store
        const uint32_t i = tid < NX * nsb * 4 ? tid : 0;
        const uint32_t p = i / (nsb * 4), rem = i % (nsb * 4), sb = rem >> 2, cc = rem & 3;
        const uint32_t pp = p < nx ? p : 0;
        const uint8_t * xb = ks_xsb<FMT>((const uint8_t *)col_pick<NX>(C.x, pp), cols, sb);
        u32x4a v[4];
        uint32_t bs[4], dkb;
        ks_xrec_issue<FMT>(xb, cc, v, bs, dkb);
        ks_wait_behind<NI, D + 1>(after_loads());
        KS_STAMP(5);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            xfence(v[k]);
            xfence(bs[k]);
        }
        xfence(dkb);
        if constexpr (FMT == FMT_Q6_K) {
#pragma unroll
            for (int k = 0; k < 4; ++k) bs[k] = (uint32_t)(32 * (int)bs[k]);
        }
        if (tid < NX * nsb * 4) {
            uint8_t * rec = xr + (size_t)tid * XREC;
#pragma unroll
            for (int k = 0; k < 4; ++k) lds_st128(rec + 16 * k, v[k]);
            lds_st128(rec + 64, u32x4a{bs[0], bs[1], bs[2], bs[3]});
            if constexpr (FMT == FMT_Q8_0) {
                lds_st32(&xd[(p * nsb + sb) * 8 + 2 * cc], __float_as_uint((p < nx) ? h2f(bs[0]) : 0.f));
                lds_st32(&xd[(p * nsb + sb) * 8 + 2 * cc + 1], __float_as_uint((p < nx) ? h2f(bs[1]) : 0.f));
            } else if (cc == 0) {
                lds_st32(&xd[p * nsb + sb], (p < nx) ? dkb : 0u);
            }
        }
    } else {
        for (uint32_t i = tid; i < NX * nsb * 4; i += blockDim.x) {
            const uint32_t p = i / (nsb * 4), rem = i % (nsb * 4), sb = rem >> 2, cc = rem & 3;
            const uint32_t pp = p < nx ? p : 0;
            const uint8_t * xb = ks_xsb<FMT>((const uint8_t *)col_pick<NX>(C.x, pp), cols, sb);
            uint8_t * rec = xr + (size_t)i * XREC;
            u32x4a v[4];
            uint32_t bs[4], dkb;
            ks_xrec_issue<FMT>(xb, cc, v, bs, dkb);
            WAIT_VM(0);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                xfence(v[k]);
                xfence(bs[k]);
            }
            xfence(dkb);
            if constexpr (FMT == FMT_Q6_K) {
#pragma unroll
                for (int k = 0; k < 4; ++k) bs[k] = (uint32_t)(32 * (int)bs[k]);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) lds_st128(rec + 16 * k, v[k]);
            lds_st128(rec + 64, u32x4a{bs[0], bs[1], bs[2], bs[3]});
            if constexpr (FMT == FMT_Q8_0) {
                lds_st32(&xd[(p * nsb + sb) * 8 + 2 * cc], __float_as_uint((p < nx) ? h2f(bs[0]) : 0.f));
                lds_st32(&xd[(p * nsb + sb) * 8 + 2 * cc + 1], __float_as_uint((p < nx) ? h2f(bs[1]) : 0.f));
            } else if (cc == 0) {
                lds_st32(&xd[p * nsb + sb], (p < nx) ? dkb : 0u);
            }
        }
        after_loads();
    }
}

// Integer partials of superblock s, part c of the chunk staged at st (mis =
// the chunk's global address mod 16, used by Q6_K's 2-byte-aligned blocks).
// ia / im: scale-weighted nibble dot and (Q4_K) min term per column; tag: the
// superblock's f16 d (| dmin << 16 for Q4_K).
template <int FMT, int NX, bool XREG>
__device__ __forceinline__ void ks_chunk(const uint8_t * st, uint32_t mis, uint32_t s, uint32_t c,
                                         const uint8_t * xrec, uint32_t nsb, const u32x4a (&xregs)[NX][5],
                                         int (&ia)[NX], int (&im)[NX], uint32_t & tag) {
    if constexpr (FMT == FMT_Q8_0) {
        // blocks 2c, 2c + 1 of unit s: 68 bytes at a 4-byte aligned offset
        const uint32_t * u = (const uint32_t *)(st + 272 * s + 68 * c);
        uint32_t w[17];
#pragma unroll
        for (int i = 0; i < 17; ++i) w[i] = u[i];
        tag = (w[0] & 0xFFFFu) | (w[8] & 0xFFFF0000u);       // d of block 2c | d of block 2c+1 << 16
        int q0[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q0[i] = (int)alignb(w[i + 1], w[i], 2);
#pragma unroll
        for (int p = 0; p < NX; ++p) {
            const uint8_t * xp = xrec + (size_t)p * nsb * 4 * XREC;
            u32x4a xv[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if constexpr (XREG) xv[k] = xregs[p][k]; else xv[k] = *(const u32x4a *)(xp + 16 * k);
            }
            int d0 = 0, d1 = 0;
            d0 = dot4(q0[0], (int)xv[0].x, d0); d0 = dot4(q0[1], (int)xv[0].y, d0);
            d0 = dot4(q0[2], (int)xv[0].z, d0); d0 = dot4(q0[3], (int)xv[0].w, d0);
            d0 = dot4(q0[4], (int)xv[1].x, d0); d0 = dot4(q0[5], (int)xv[1].y, d0);
            d0 = dot4(q0[6], (int)xv[1].z, d0); d0 = dot4(q0[7], (int)xv[1].w, d0);
            d1 = dot4((int)w[9], (int)xv[2].x, d1); d1 = dot4((int)w[10], (int)xv[2].y, d1);
            d1 = dot4((int)w[11], (int)xv[2].z, d1); d1 = dot4((int)w[12], (int)xv[2].w, d1);
            d1 = dot4((int)w[13], (int)xv[3].x, d1); d1 = dot4((int)w[14], (int)xv[3].y, d1);
            d1 = dot4((int)w[15], (int)xv[3].z, d1); d1 = dot4((int)w[16], (int)xv[3].w, d1);
            ia[p] = d0;
            im[p] = d1;
        }
    } else if constexpr (FMT == FMT_Q4_K) {
        const u32x4a hd = *(const u32x4a *)(st + 144 * s);
        const u32x4a qa = *(const u32x4a *)(st + 144 * s + 16 + 16 * c);
        const u32x4a qb = *(const u32x4a *)(st + 144 * s + 80 + 16 * c);
        tag = hd.x;
        const uint32_t sclo = hd.y & 0x3F3F3F3Fu, mlo = hd.z & 0x3F3F3F3Fu;
        const uint32_t schi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t mhi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
        const uint32_t sh = (c >> 1) * 16;
        const int sc[4] = {(int)((sclo >> sh) & 0xFF), (int)((sclo >> (sh + 8)) & 0xFF),
                           (int)((schi >> sh) & 0xFF), (int)((schi >> (sh + 8)) & 0xFF)};
        const int mn[4] = {(int)((mlo >> sh) & 0xFF), (int)((mlo >> (sh + 8)) & 0xFF),
                           (int)((mhi >> sh) & 0xFF), (int)((mhi >> (sh + 8)) & 0xFF)};
        const uint32_t q[2][4] = {{qa.x, qa.y, qa.z, qa.w}, {qb.x, qb.y, qb.z, qb.w}};
        int nib[4][4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            nib[0][k] = (int)(q[0][k] & 0x0F0F0F0Fu);
            nib[1][k] = (int)((q[0][k] >> 4) & 0x0F0F0F0Fu);
            nib[2][k] = (int)(q[1][k] & 0x0F0F0F0Fu);
            nib[3][k] = (int)((q[1][k] >> 4) & 0x0F0F0F0Fu);
        }
#pragma unroll
        for (int p = 0; p < NX; ++p) {
            const uint8_t * xp = xrec + (size_t)p * nsb * 4 * XREC;
            int acc_i = 0;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                u32x4a xv;
                if constexpr (XREG) xv = xregs[p][g]; else xv = *(const u32x4a *)(xp + 16 * g);
                int d = 0;
                d = dot4(nib[g][0], (int)xv.x, d);
                d = dot4(nib[g][1], (int)xv.y, d);
                d = dot4(nib[g][2], (int)xv.z, d);
                d = dot4(nib[g][3], (int)xv.w, d);
                acc_i += sc[g] * d;
            }
            u32x4a bsv;
            if constexpr (XREG) bsv = xregs[p][4]; else bsv = *(const u32x4a *)(xp + 64);
            ia[p] = acc_i;
            im[p] = mn[0] * (int)bsv.x + mn[1] * (int)bsv.y + mn[2] * (int)bsv.z + mn[3] * (int)bsv.w;
        }
    } else {
        const uint32_t so = mis + 210 * s;
        const uint32_t hh = c >> 1, bb = c & 1;
        uint32_t A[4], Bq[4], H[4], S[4];
        lds16_u2(st, so + 64 * hh + 16 * bb, A);
        lds16_u2(st, so + 64 * hh + 32 + 16 * bb, Bq);
        lds16_u2(st, so + 128 + 32 * hh + 16 * bb, H);
        lds16_u2(st, so + 192, S);
        const uint32_t dw = *(const uint32_t *)(st + ((so + 208) & ~3u));
        tag = ((so + 208) & 2u) ? (dw >> 16) : (dw & 0xFFFFu);
        const uint32_t sd0 = hh ? S[2] : S[0], sd1 = hh ? S[3] : S[1];
        const int sc[4] = {(int)(int8_t)(sd0 >> (8 * bb)), (int)(int8_t)(sd0 >> (8 * bb + 16)),
                           (int)(int8_t)(sd1 >> (8 * bb)), (int)(int8_t)(sd1 >> (8 * bb + 16))};
        int g6[4][4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            g6[0][k] = (int)((A[k] & 0x0F0F0F0Fu) | ((H[k] & 0x03030303u) << 4));
            g6[1][k] = (int)((Bq[k] & 0x0F0F0F0Fu) | ((H[k] << 2) & 0x30303030u));
            g6[2][k] = (int)(((A[k] >> 4) & 0x0F0F0F0Fu) | (H[k] & 0x30303030u));
            g6[3][k] = (int)(((Bq[k] >> 4) & 0x0F0F0F0Fu) | ((H[k] >> 2) & 0x30303030u));
        }
#pragma unroll
        for (int p = 0; p < NX; ++p) {
            const uint8_t * xp = xrec + (size_t)p * nsb * 4 * XREC;
            u32x4a bsv;
            if constexpr (XREG) bsv = xregs[p][4]; else bsv = *(const u32x4a *)(xp + 64);
            const int b32[4] = {(int)bsv.x, (int)bsv.y, (int)bsv.z, (int)bsv.w};
            int acc_i = 0;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                u32x4a xv;
                if constexpr (XREG) xv = xregs[p][g]; else xv = *(const u32x4a *)(xp + 16 * g);
                int d = 0;
                d = dot4(g6[g][0], (int)xv.x, d);
                d = dot4(g6[g][1], (int)xv.y, d);
                d = dot4(g6[g][2], (int)xv.z, d);
                d = dot4(g6[g][3], (int)xv.w, d);
                acc_i += sc[g] * (d - b32[g]);
            }
            ia[p] = acc_i;
            im[p] = 0;
        }
    }
}

// Quad-reduce the partials and park them as (row rl, column p, superblock sb)
// terms (lane c == 0 of each quad writes).
template <int FMT, int NX>
__device__ __forceinline__ void ks_park(int (&ia)[NX], int (&im)[NX], uint32_t tag, bool act, uint32_t c,
                                        uint32_t nx, uint32_t rl, uint32_t sb, uint32_t nsb,
                                        int * TI, int * TM, uint32_t * TH) {
    if constexpr (FMT == FMT_Q8_0) {       // exact per-block sums, no reduction: every lane parks two
        const uint32_t nb = nsb * 8, b = 8 * sb + 2 * c;
#pragma unroll
        for (int p = 0; p < NX; ++p) {
            if (act && p < (int)nx) {
                TI[(rl * NX + p) * nb + b] = ia[p];
                TI[(rl * NX + p) * nb + b + 1] = im[p];
            }
        }
        if (act) {
            TH[rl * nb + b] = tag & 0xFFFFu;
            TH[rl * nb + b + 1] = tag >> 16;
        }
        return;
    }
#pragma unroll
    for (int p = 0; p < NX; ++p) {
        int x1 = ia[p];
        x1 += qx1(x1); x1 += qx2(x1);
        if (act && c == 0 && p < (int)nx) TI[(rl * NX + p) * nsb + sb] = x1;
        if constexpr (FMT == FMT_Q4_K) {
            int m1 = im[p];
            m1 += qx1(m1); m1 += qx2(m1);
            if (act && c == 0 && p < (int)nx) TM[(rl * NX + p) * nsb + sb] = m1;
        }
    }
    if (act && c == 0) TH[rl * nsb + sb] = tag;
}

// Reference-order fold of row rl, column p: lane k (0..3) runs accumulator k
// over superblocks k, k+4, ...; the quad then combines (a0 + a1) + (a2 + a3).
template <int FMT, int NX>
__device__ __forceinline__ float ks_fold(const int * TI, const int * TM, const uint32_t * TH, const float * xd,
                                         uint32_t nsb, uint32_t k, uint32_t p, uint32_t rl, bool fok) {
    float acc = 0.f;
    if constexpr (FMT == FMT_Q8_0) {       // acc[b & 3] over 32-weight blocks (fl_dot_i8_q8_0 order)
        if (fok) {
            const uint32_t nb = nsb * 8;
            const int * ti = TI + (rl * NX + p) * nb;
            const uint32_t * th = TH + rl * nb;
            const float * xdp = xd + p * nb;
            for (uint32_t b = k; b < nb; b += 4) acc = fmaf(h2f(th[b]) * xdp[b], (float)ti[b], acc);
        }
        const float s01 = acc + qx1f(acc);
        return s01 + qx2f(s01);
    }
    if (fok) {
        const int * ti = TI + (rl * NX + p) * nsb;
        const int * tm = TM + (rl * NX + p) * nsb;
        const uint32_t * th = TH + rl * nsb;
        const float * xdp = xd + p * nsb;
        auto step = [&](uint32_t sbi) {
            const float dk = xdp[sbi];
            if constexpr (FMT == FMT_Q4_K) {
                const float d = h2f(th[sbi] & 0xFFFFu), dmin = h2f(th[sbi] >> 16);
                acc = fmaf(d * dk, (float)ti[sbi], acc);
                acc = fmaf(-(dmin * dk), (float)tm[sbi], acc);
            } else {
                acc = fmaf(h2f(th[sbi]) * dk, (float)ti[sbi], acc);
            }
        };
        // four steps per iteration so their loads are issued together
        uint32_t sbi = k;
        for (; sbi + 12 < nsb; sbi += 16) {
#pragma unroll
            for (int q = 0; q < 4; ++q) step(sbi + 4 * q);
        }
        for (; sbi < nsb; sbi += 4) step(sbi);
    }
    const float s01 = acc + qx1f(acc);
    return s01 + qx2f(s01);
}

// Expert ids of the ntok * top_k routed pairs for a grouped expert matvec:
// a.ids, or with a fused ROUTER_SEL (a.rt_logits) the ids this workgroup
// computes into rids (LDS, ntok * top_k entries), one wave per token;
// workgroup (0, 0) also publishes ids and gates.  Contains a barrier.
__device__ __forceinline__ const uint32_t * moe_route(const MoeArgs & a, uint32_t * rids) {
    if (!a.rt_logits) return a.ids;
    const uint32_t lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    const bool pub = blockIdx.x == 0 && blockIdx.y == 0;
    for (uint32_t t = threadIdx.x >> 6; t < a.ntok; t += nw)
        router_token_wave(a.rt_logits + (size_t)t * a.n_expert, a.n_expert, a.top_k, a.rt_norm, a.rt_scale, lane,
                          rids + (size_t)t * a.top_k, pub ? a.rt_gates + (size_t)t * a.top_k : nullptr);
    __syncthreads();
    if (pub)
        for (uint32_t i = threadIdx.x; i < a.ntok * a.top_k; i += blockDim.x) ((uint32_t *)a.ids)[i] = rids[i];
    return rids;
}

// Work of grouped-matvec workgroup b of B (flattened grid): the n routed
// experts (distinct ids among the nids pairs) share the B workgroups evenly,
// expert j (the j-th smallest id) taking workgroups [ceil(jB/n),
// ceil((j+1)B/n)); returns e = n_expert when nothing is routed, else e and
// this workgroup's index g among its expert's G.  Every workgroup computes the
// same split from the same ids, so none idles on an unrouted expert.
// Contains barriers.
__device__ __forceinline__ uint32_t moe_assign(const uint32_t * ids, uint32_t nids, uint32_t n_expert, uint32_t b,
                                               uint32_t B, uint32_t & g, uint32_t & G) {
    __shared__ uint32_t em[8];
    __shared__ uint32_t pick;
    if (threadIdx.x < 8) em[threadIdx.x] = 0u;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < nids; i += blockDim.x) {
        const uint32_t e = ids[i];
        if (e < n_expert && e < 256) atomicOr(&em[e >> 5], 1u << (e & 31));
    }
    __syncthreads();
    uint32_t n = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) n += (uint32_t)__popc(em[w]);
    const uint32_t j = n ? b * n / B : 0u;                  // b * n < 2^32: B <= 2^20 workgroups
    if (threadIdx.x == 0) {
        uint32_t k = j, r = n_expert;
        for (uint32_t w = 0; w < 8 && r == n_expert && n; ++w) {
            uint32_t m = em[w];
            const uint32_t c = (uint32_t)__popc(m);
            if (k < c) {
                for (; k; --k) m &= m - 1;
                r = 32 * w + (uint32_t)__ffs(m) - 1;
            } else {
                k -= c;
            }
        }
        pick = r;
    }
    __syncthreads();
    const uint32_t nn = n ? n : 1u;
    const uint32_t s0 = (j * B + nn - 1) / nn, s1 = ((j + 1) * B + nn - 1) / nn;
    g = b - s0;
    G = s1 - s0;
    return pick;
}

}  // namespace flh
