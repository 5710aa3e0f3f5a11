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

__device__ __forceinline__ uint32_t ks_quant16(const u32x4a (&raw)[4], float id, int & sum, uint32_t (&pk)[4]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t r4[4] = {raw[k].x, raw[k].y, raw[k].z, raw[k].w};
        pk[k] = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float qv = roundf(__uint_as_float(r4[j]) * id);
            if (qv > 127.f) qv = 127.f;
            if (qv < -127.f) qv = -127.f;
            sum += (int)qv;
            pk[k] |= ((uint32_t)(int)qv & 0xFFu) << (8 * j);
        }
    }
    return 0;
}

__device__ __forceinline__ float ks_absmax16(const u32x4a (&raw)[4]) {
    float m = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        m = fmaxf(fmaxf(fmaxf(m, fabsf(__uint_as_float(raw[k].x))), fabsf(__uint_as_float(raw[k].y))),
                  fmaxf(fabsf(__uint_as_float(raw[k].z)), fabsf(__uint_as_float(raw[k].w))));
    return m;
}

// ACT_Q8 fused into the dot: quantise the fp32 columns into the records
// (16 lanes per superblock, each lane one 16-element run).  When write_app,
// also write both appendices so the bytes in memory equal ACT_Q8's.  A
// superblock's 16 runs sit in 16 consecutive lanes of one wave, so its absmax
// is a 4-step shuffle max (order-free), with no barrier.  after_loads() runs
// once, right after the first activation loads are issued (the caller issues
// its weight prologue there, behind the older activation loads).
template <int FMT, int NX, int KW = 4, typename F>
__device__ __forceinline__ void ks_x_fuse(const KsCols<NX> & C, uint32_t nx, uint32_t nsb, uint32_t cols,
                                          uint8_t * xr, float * xd, bool write_app, F && after_loads) {
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nitem = nx * nsb;
    const uint32_t sub = lane >> 4, run = lane & 15;        // superblock in the pass, 16-run
    bool issued = false;
    for (uint32_t base = 0; base < nitem; base += 16 * KW) {
        // up to 16 KW superblocks per pass (4 KW per q-group, 4 per wave),
        // loads first; only the q-groups that hold superblocks are loaded
        const uint32_t nq = min(4u, (nitem - base + 4 * KW - 1) / (4 * KW));
        u32x4a raw[4][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if ((uint32_t)q >= nq) break;
            const uint32_t i = base + 4 * KW * q + 4 * wave + sub;
            const uint32_t ii = i < nitem ? i : 0;
            const float * src = col_pick<NX>(C.x, ii / nsb) + 256 * (ii % nsb) + 16 * run;
#pragma unroll
            for (int k = 0; k < 4; ++k) raw[q][k] = *(const u32x4a *)(src + 4 * k);
        }
        if (!issued) {
            after_loads();
            issued = true;
        }
        // superblock absmax: its 16 runs are 16 consecutive lanes of this wave
        float amq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if ((uint32_t)q >= nq) break;                   // wave-uniform
            float m = ks_absmax16(raw[q]);
            m = fmaxf(m, __shfl_xor(m, 1));
            m = fmaxf(m, __shfl_xor(m, 2));
            m = fmaxf(m, __shfl_xor(m, 4));
            amq[q] = fmaxf(m, __shfl_xor(m, 8));
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t i = base + 4 * KW * q + 4 * wave + sub;
            if ((uint32_t)q < nq && i < nitem) {
                const uint32_t p = i / nsb, sb = i % nsb;
                const float amax = amq[q];
                const float d = amax / 127.f;
                const float id = amax > 0.f ? 127.f / amax : 0.f;
                uint32_t pk[4];
                int sum = 0;
                ks_quant16(raw[q], id, sum, pk);
                uint32_t cc, kk, t;
                xrec_pos<FMT>(16 * run, cc, kk, t);
                uint8_t * rec = xr + (((size_t)p * nsb + sb) * 4 + cc) * XREC;
                lds_st128(rec + 16 * kk, u32x4a{pk[0], pk[1], pk[2], pk[3]});
                lds_st32(rec + 64 + 4 * kk, (uint32_t)(FMT == FMT_Q4_K ? sum : 32 * sum));
                if (run == 0) lds_st32(&xd[p * nsb + sb], __float_as_uint(d));
                if (write_app) {
                    float * xc = (float *)col_pick<NX>(C.x, p);
                    uint8_t * q8k = (uint8_t *)xc + xqk_off(cols) + (size_t)sb * 292;
                    uint32_t * dst = (uint32_t *)(q8k + 36 + 16 * run);
#pragma unroll
                    for (int k = 0; k < 4; ++k) dst[k] = pk[k];
                    *(int16_t *)(q8k + 4 + 2 * run) = (int16_t)sum;
                    if (run == 0) *(float *)q8k = d;
                    // q8_1 block of 32 = this lane's run and its neighbour's
                    float m2 = ks_absmax16(raw[q]);
                    m2 = fmaxf(m2, __shfl_xor(m2, 1));
                    const float d1 = m2 / 127.f;
                    const float id1 = m2 > 0.f ? 127.f / m2 : 0.f;
                    uint32_t pk1[4];
                    int s1 = 0;
                    ks_quant16(raw[q], id1, s1, pk1);
                    s1 += __shfl_xor(s1, 1);
                    uint8_t * q81 = (uint8_t *)xc + xq_off(cols) + (size_t)(sb * 8 + (run >> 1)) * 36;
                    uint32_t * d1p = (uint32_t *)(q81 + 4 + 16 * (run & 1));
#pragma unroll
                    for (int k = 0; k < 4; ++k) d1p[k] = pk1[k];
                    if ((run & 1) == 0) *(uint32_t *)q81 = f2h(d1) | (f2h(d1 * (float)s1) << 16);
                }
            }
        }
    }
    if (!issued) after_loads();
    // columns p >= nx of the template width read zero records
    for (uint32_t i = tid; i < (NX - nx) * nsb * 4 * (XREC / 4); i += 256)
        ((uint32_t *)(xr + (size_t)nx * nsb * 4 * XREC))[i] = 0u;
    for (uint32_t i = tid; i < (NX - nx) * nsb; i += 256) xd[nx * nsb + i] = 0.f;
}

// Record (sb, part cc) of column p from its appendix at xb (the superblock's
// base: q8_K for the K formats; for Q8_0, the unit's 8 q8_1 blocks, whose
// scales go to bs[0..1] as raw halves).
template <int FMT>
__device__ __forceinline__ void ks_xrec_load(const uint8_t * xb, uint32_t cc, u32x4 (&v)[4], int (&bs)[4]) {
    if constexpr (FMT == FMT_Q8_0) {
        const uint8_t * b0 = xb + 72 * cc;                  // q8_1 blocks 2cc, 2cc + 1 (36 B each)
        v[0] = ld4(b0 + 4);
        v[1] = ld4(b0 + 20);
        v[2] = ld4(b0 + 40);
        v[3] = ld4(b0 + 56);
        bs[0] = (int)*(const uint16_t *)b0;
        bs[1] = (int)*(const uint16_t *)(b0 + 36);
        bs[2] = bs[3] = 0;
    } else if constexpr (FMT == FMT_Q4_K) {
        const uint32_t g0 = 2 * (cc >> 1), h = cc & 1;
        const uint32_t gs[4] = {g0, g0 + 1, g0 + 4, g0 + 5};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[k] = ld4(xb + 36 + 32 * gs[k] + 16 * h);
            bs[k] = *(const int16_t *)(xb + 4 + 2 * (2 * gs[k] + h));
        }
    } else {
        const uint32_t hh = cc >> 1, bb = cc & 1;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            v[g] = ld4(xb + 36 + 128 * hh + 32 * g + 16 * bb);
            bs[g] = 32 * (int)*(const int16_t *)(xb + 4 + 2 * (8 * hh + 2 * g + bb));
        }
    }
}

// Base of superblock sb's activation in column x: its q8_K block (K formats)
// or its 8 q8_1 blocks (Q8_0).
template <int FMT>
__device__ __forceinline__ const uint8_t * ks_xsb(const uint8_t * x, uint32_t cols, uint32_t sb) {
    return FMT == FMT_Q8_0 ? x + xq_off(cols) + (size_t)sb * 288 : x + xqk_off(cols) + (size_t)sb * 292;
}

// Records from the appendices written by ACT_Q8.  after_loads() as above.
template <int FMT, int NX, typename F>
__device__ __forceinline__ void ks_x_app(const KsCols<NX> & C, uint32_t nx, uint32_t nsb, uint32_t cols,
                                         uint8_t * xr, float * xd, F && after_loads) {
    const uint32_t tid = threadIdx.x;
    if (NX * nsb * 4 <= 256) {
        // one record per thread: load, run after_loads, then store
        const uint32_t i = tid < NX * nsb * 4 ? tid : 0;
        const uint32_t p = i / (nsb * 4), rem = i % (nsb * 4), sb = rem >> 2, cc = rem & 3;
        const uint32_t pp = p < nx ? p : 0;
        const uint8_t * xb = ks_xsb<FMT>((const uint8_t *)col_pick<NX>(C.x, pp), cols, sb);
        u32x4 v[4];
        int bs[4];
        ks_xrec_load<FMT>(xb, cc, v, bs);
        const float dk = FMT == FMT_Q8_0 ? 0.f : *(const float *)xb;
        after_loads();
        if (tid < NX * nsb * 4) {
            uint8_t * rec = xr + (size_t)tid * XREC;
#pragma unroll
            for (int k = 0; k < 4; ++k) lds_st128(rec + 16 * k, u32x4a{v[k].x, v[k].y, v[k].z, v[k].w});
            lds_st128(rec + 64, u32x4a{(uint32_t)bs[0], (uint32_t)bs[1], (uint32_t)bs[2], (uint32_t)bs[3]});
            if constexpr (FMT == FMT_Q8_0) {
                lds_st32(&xd[(p * nsb + sb) * 8 + 2 * cc], __float_as_uint((p < nx) ? h2f((uint32_t)bs[0]) : 0.f));
                lds_st32(&xd[(p * nsb + sb) * 8 + 2 * cc + 1], __float_as_uint((p < nx) ? h2f((uint32_t)bs[1]) : 0.f));
            } else if (cc == 0) {
                lds_st32(&xd[p * nsb + sb], __float_as_uint((p < nx) ? dk : 0.f));
            }
        }
    } else {
        for (uint32_t i = tid; i < NX * nsb * 4; i += 256) {
            const uint32_t p = i / (nsb * 4), rem = i % (nsb * 4), sb = rem >> 2, cc = rem & 3;
            const uint32_t pp = p < nx ? p : 0;
            const uint8_t * xb = ks_xsb<FMT>((const uint8_t *)col_pick<NX>(C.x, pp), cols, sb);
            uint32_t * rec = (uint32_t *)(xr + (size_t)i * XREC);
            u32x4 v[4];
            int bs[4];
            ks_xrec_load<FMT>(xb, cc, v, bs);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                rec[4 * k + 0] = v[k].x; rec[4 * k + 1] = v[k].y; rec[4 * k + 2] = v[k].z; rec[4 * k + 3] = v[k].w;
                rec[16 + k] = (uint32_t)bs[k];
            }
            if constexpr (FMT == FMT_Q8_0) {
                xd[(p * nsb + sb) * 8 + 2 * cc] = (p < nx) ? h2f((uint32_t)bs[0]) : 0.f;
                xd[(p * nsb + sb) * 8 + 2 * cc + 1] = (p < nx) ? h2f((uint32_t)bs[1]) : 0.f;
            } else if (cc == 0) {
                xd[p * nsb + sb] = (p < nx) ? *(const float *)xb : 0.f;
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

// ---------------------------------------------------------------- ACT_Q8 --
// One wave quantises one 256-element chunk: lane i holds elements 4i..4i+3
// in v.  Writes the chunk's q8_1 blocks (8-lane groups) and its q8_K block
// with the bytes of fl_quantize_q8_1_block / fl_quantize_q8_K_block
// (src/runtime/quants.h:360-402): amax is a max (order free), d = amax/127
// and id = 127/amax are correctly rounded IEEE divisions, q = roundf(x*id)
// clamped to +-127, sums are exact integers, halves are RNE.
__device__ __forceinline__ float wave_max8(float v) {      // within 8 lanes
    v = fmaxf(v, __shfl_xor(v, 1));
    v = fmaxf(v, __shfl_xor(v, 2));
    v = fmaxf(v, __shfl_xor(v, 4));
    return v;
}
__device__ __forceinline__ int isum8(int v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    return v;
}
__device__ __forceinline__ uint32_t quant4(const float (&v)[4], float id, int & sum) {
    uint32_t packed = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float q = roundf(v[j] * id);
        if (q > 127.f) q = 127.f;
        if (q < -127.f) q = -127.f;
        const int qi = (int)q;
        sum += qi;
        packed |= ((uint32_t)qi & 0xFFu) << (8 * j);
    }
    return packed;
}
__device__ __forceinline__ void act_q8_lanes(const float (&v)[4], uint32_t lane, uint32_t chunk,
                                             uint8_t * q81, uint8_t * q8k, uint32_t cols) {
    const float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    // q8_1: block of 32 = 8 lanes
    {
        const uint32_t blk = chunk * 8 + (lane >> 3);
        const float amax = wave_max8(am);
        const float d = amax / 127.f;
        const float id = amax > 0.f ? 127.f / amax : 0.f;
        int s = 0;
        const uint32_t pk = quant4(v, id, s);
        const int sum = isum8(s);
        if ((blk + 1) * 32 <= cols) {
            uint8_t * o = q81 + (size_t)blk * 36;
            *(uint32_t *)(o + 4 + 4 * (lane & 7)) = pk;
            if ((lane & 7) == 0) *(uint32_t *)o = f2h(d) | (f2h(d * (float)sum) << 16);
        }
    }
    // q8_K: whole chunk
    if ((chunk + 1) * 256 <= cols) {
        float amax = wave_max8(am);
        amax = fmaxf(amax, __shfl_xor(amax, 8));
        amax = fmaxf(amax, __shfl_xor(amax, 16));
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        const float d = amax / 127.f;
        const float id = amax > 0.f ? 127.f / amax : 0.f;
        int s = 0;
        const uint32_t pk = quant4(v, id, s);
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        uint8_t * o = q8k + (size_t)chunk * 292;
        *(uint32_t *)(o + 36 + 4 * lane) = pk;
        if ((lane & 3) == 0) *(int16_t *)(o + 4 + 2 * (lane >> 2)) = (int16_t)s;
        if (lane == 0) *(float *)o = d;
    }
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
