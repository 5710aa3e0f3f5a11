// flh_dot_kstream.hip -- LDS-staged int8 x q8_K row-dots for Q4_K / Q6_K.
//
// The streamed weight bytes go HBM -> LDS with gfx950's direct-to-LDS
// dwordx4 loads (global_load_lds_dwordx4), one fully coalesced pass: every
// 64-byte line of the matrix is requested from L2 exactly once.  (Loading a
// superblock's header and nibbles straight into the lanes that use them asks
// L2 for each line ~3x, and that request rate, not HBM, becomes the limit.)
//
// Work unit: a CHUNK of 16 consecutive superblocks of the row-major matrix
// (rows are contiguous, so a chunk may straddle a row boundary).  A workgroup
// (4 waves) owns a batch of nr whole rows; its chunks are dealt round-robin
// to the waves, each wave keeping D chunks in flight in a private LDS ring.
// Lane (slot s = lane/4, part c = lane%4) of a wave handles superblock s of
// the chunk, quarter c, exactly as in flh_dot_int8.hip: integer partials,
// DPP quad reduction, (row, column, superblock) terms parked in LDS, then the
// reference-order float fold per (row, column, accumulator).  Results are
// bitwise equal to fl_dot_i8k_q4_K / fl_dot_i8k_q6_K
// (src/runtime/quants.h:538-594).
//
// The activation (q8_K appendix) is re-laid in LDS once per workgroup as
// 80-byte per-lane records (64 int8 + 4 int32 block sums), so every lane
// reads its slice with five conflict-free 16-byte LDS reads.
#include "flh_common.h"
#include "flh_internal.h"
#include "flh_status.h"
#include <stdio.h>
#include <stdlib.h>

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

constexpr uint32_t XREC = 80;                        // bytes per (sb, part) activation record

template <int FMT>
__host__ __device__ inline size_t ks_smem_bytes(uint32_t nr, uint32_t nx, uint32_t nsb, int D) {
    const size_t stages = (size_t)4 * D * KS<FMT>::WIN;
    const size_t xrec = (size_t)nx * nsb * 4 * XREC + (size_t)nx * nsb * 4;
    const size_t terms = (size_t)nr * nx * nsb * 4 * (FMT == FMT_Q4_K ? 2 : 1) + (size_t)nr * nsb * 4;
    return stages + xrec + terms;
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

__device__ __forceinline__ void wait_vm_upto(uint32_t n) {
    switch (n) {
        case 0: WAIT_VM(0); break;
        case 3: WAIT_VM(3); break;
        case 4: WAIT_VM(4); break;
        case 6: WAIT_VM(6); break;
        case 8: WAIT_VM(8); break;
        case 9: WAIT_VM(9); break;
        case 12: WAIT_VM(12); break;
        default: WAIT_VM(0); break;
    }
}

typedef uint32_t u32x4a __attribute__((ext_vector_type(4)));

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

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}

// Columns of one kstream pass: x_p / y_p base pointers (p < nx <= NX).
template <int NX>
struct KsCols {
    const float * x[NX];
    float * y[NX];
};
// runtime column select without dynamic register indexing
template <int NX, typename T>
__device__ __forceinline__ T col_pick(T const (&v)[NX], uint32_t p) {
    T r = v[0];
#pragma unroll
    for (int i = 1; i < NX; ++i) r = p == (uint32_t)i ? v[i] : r;
    return r;
}

// One pass over rows [0, rows) of the matrix at w for nx <= NX columns; the
// workgroup owns batches batch0, batch0 + G, ...  Ends with every weight DMA
// drained, so the caller may start another pass on the same LDS.
template <int FMT, int NX, int D, bool FUSE, bool XREG>
__device__ __forceinline__ void ks_body(const uint8_t * __restrict__ w, uint32_t rows, uint32_t cols,
                                        const KsCols<NX> & C, uint32_t nx, uint32_t nr,
                                        uint32_t batch0, uint32_t G, uint8_t * sm) {
    constexpr uint32_t B = KS<FMT>::BLK, WIN = KS<FMT>::WIN;
    constexpr int NI = KS<FMT>::NI;
    const uint32_t nsb = cols >> 8;
    const uint64_t rb = (uint64_t)nsb * B;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    // wave-uniform: keeps the chunk cursor and batch logic on the scalar unit
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t s = lane >> 2, c = lane & 3;

    uint8_t * stages = sm;                                        // [4][D][WIN]
    uint8_t * xr = sm + (size_t)4 * D * WIN;                      // [NX][nsb][4][80]
    float * xd = (float *)(xr + (size_t)NX * nsb * 4 * XREC);     // [NX][nsb]
    int * TI = (int *)(xd + (size_t)NX * nsb);                    // [nr][NX][nsb]
    int * TM = TI + (size_t)nr * NX * nsb;                        // Q4_K only
    uint32_t * TH = (uint32_t *)(FMT == FMT_Q4_K ? TM + (size_t)nr * NX * nsb : TM);   // [nr][nsb]
    uint8_t * myst = stages + (size_t)wave * D * WIN;

    const uint32_t nbatch = (rows + nr - 1) / nr;
    auto nci_of = [&](uint32_t bt) -> uint32_t {                  // this wave's chunks in batch bt
        const uint32_t nrow = min(nr, rows - bt * nr);
        const uint32_t nch = (nrow * nsb + 15) / 16;
        return nch > wave ? (nch - wave + 3) / 4 : 0;
    };
    // Issue cursor over this wave's chunk sequence (batches blockIdx.x, +G, ...).
    // Every call issues exactly NI loads (a repeat of the last real chunk once
    // the sequence is exhausted), so the count of loads behind any chunk is
    // always NI * (D - 1).
    uint32_t qbt = batch0, qci = 0, qn = qbt < nbatch ? nci_of(qbt) : 0;
    const uint8_t * l_wb = w;            // a wave without chunks re-reads row 0 (valid, unused)
    uint32_t l_ch = 0, l_nsbb = nsb;
    auto issue_one = [&](uint8_t * stage) {
        while (qbt < nbatch && qci >= qn) {
            qbt += G;
            qci = 0;
            qn = qbt < nbatch ? nci_of(qbt) : 0;
        }
        if (qbt < nbatch) {
            l_wb = w + (size_t)qbt * nr * rb;
            l_ch = wave + 4 * qci;
            l_nsbb = min(nr, rows - qbt * nr) * nsb;
            ++qci;
        }
        ks_issue<FMT>(l_wb, l_ch, l_nsbb, stage, lane);
    };
    // The first D weight chunks are issued right after the activation loads
    // (which are older, so waiting for them does not wait for the weights).
    auto prologue = [&]() {
#pragma unroll
        for (int j = 0; j < D; ++j) issue_one(myst + j * WIN);
    };
    bool issued = false;

    // ---- activation records, once per workgroup (overlaps the first weight DMAs)
    if constexpr (FUSE) {
        // ACT_Q8 fused: quantise the fp32 columns here (16 lanes per
        // superblock, each lane one 16-element run); workgroup 0 also writes
        // both appendices so the bytes in memory equal ACT_Q8's.  The
        // superblock absmax is an LDS atomic max over the lanes' partial
        // maxima (bit patterns of non-negative floats order like the floats).
        __shared__ uint32_t amx[64];
        const uint32_t nitem = nx * nsb;
        const uint32_t sub = lane >> 4, run = lane & 15;        // superblock in the pass, 16-run
        for (uint32_t base = 0; base < nitem; base += 64) {
            // 16 superblocks per wave-pass (4 per pass x 4 passes), loads first
            u32x4a raw[4][4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t i = base + 16 * q + 4 * wave + sub;
                const uint32_t ii = i < nitem ? i : 0;
                const float * src = col_pick<NX>(C.x, ii / nsb) + 256 * (ii % nsb) + 16 * run;
#pragma unroll
                for (int k = 0; k < 4; ++k) raw[q][k] = *(const u32x4a *)(src + 4 * k);
            }
            if (!issued) {
                prologue();
                issued = true;
            }
            if (tid < 64) amx[tid] = 0u;
            __syncthreads();
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float m = 0.f;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    m = fmaxf(fmaxf(fmaxf(m, fabsf(__uint_as_float(raw[q][k].x))), fabsf(__uint_as_float(raw[q][k].y))),
                              fmaxf(fabsf(__uint_as_float(raw[q][k].z)), fabsf(__uint_as_float(raw[q][k].w))));
                atomicMax(&amx[16 * q + 4 * wave + sub], __float_as_uint(m));
            }
            __syncthreads();
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t i = base + 16 * q + 4 * wave + sub;
                if (i < nitem) {
                    const uint32_t p = i / nsb, sb = i % nsb;
                    const float amax = __uint_as_float(amx[16 * q + 4 * wave + sub]);
                    const float d = amax / 127.f;
                    const float id = amax > 0.f ? 127.f / amax : 0.f;
                    uint32_t pk[4];
                    int sum = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint32_t r4[4] = {raw[q][k].x, raw[q][k].y, raw[q][k].z, raw[q][k].w};
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
                    uint32_t cc, kk, t;
                    xrec_pos<FMT>(16 * run, cc, kk, t);
                    uint8_t * rec = xr + (((size_t)p * nsb + sb) * 4 + cc) * XREC;
                    *(u32x4a *)(rec + 16 * kk) = u32x4a{pk[0], pk[1], pk[2], pk[3]};
                    *(int *)(rec + 64 + 4 * kk) = FMT == FMT_Q4_K ? sum : 32 * sum;
                    if (run == 0) xd[p * nsb + sb] = d;
                    if (batch0 == 0) {
                        float * xc = (float *)col_pick<NX>(C.x, p);
                        uint8_t * q8k = (uint8_t *)xc + xqk_off(cols) + (size_t)sb * 292;
                        uint32_t * dst = (uint32_t *)(q8k + 36 + 16 * run);
#pragma unroll
                        for (int k = 0; k < 4; ++k) dst[k] = pk[k];
                        *(int16_t *)(q8k + 4 + 2 * run) = (int16_t)sum;
                        if (run == 0) *(float *)q8k = d;
                        // q8_1 block of 32 = this lane's run and its neighbour's
                        float m2 = 0.f;
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            m2 = fmaxf(fmaxf(fmaxf(m2, fabsf(__uint_as_float(raw[q][k].x))), fabsf(__uint_as_float(raw[q][k].y))),
                                       fmaxf(fabsf(__uint_as_float(raw[q][k].z)), fabsf(__uint_as_float(raw[q][k].w))));
                        m2 = fmaxf(m2, __shfl_xor(m2, 1));
                        const float d1 = m2 / 127.f;
                        const float id1 = m2 > 0.f ? 127.f / m2 : 0.f;
                        uint32_t pk1[4];
                        int s1 = 0;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const uint32_t r4[4] = {raw[q][k].x, raw[q][k].y, raw[q][k].z, raw[q][k].w};
                            pk1[k] = 0;
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                float qv = roundf(__uint_as_float(r4[j]) * id1);
                                if (qv > 127.f) qv = 127.f;
                                if (qv < -127.f) qv = -127.f;
                                s1 += (int)qv;
                                pk1[k] |= ((uint32_t)(int)qv & 0xFFu) << (8 * j);
                            }
                        }
                        s1 += __shfl_xor(s1, 1);
                        uint8_t * q81 = (uint8_t *)xc + xq_off(cols) + (size_t)(sb * 8 + (run >> 1)) * 36;
                        uint32_t * d1p = (uint32_t *)(q81 + 4 + 16 * (run & 1));
#pragma unroll
                        for (int k = 0; k < 4; ++k) d1p[k] = pk1[k];
                        if ((run & 1) == 0) *(uint32_t *)q81 = f2h(d1) | (f2h(d1 * (float)s1) << 16);
                    }
                }
            }
            __syncthreads();
        }
        // columns p >= nx of the template width read zero records
        for (uint32_t i = tid; i < (NX - nx) * nsb * 4 * (XREC / 4); i += 256)
            ((uint32_t *)(xr + (size_t)nx * nsb * 4 * XREC))[i] = 0u;
        for (uint32_t i = tid; i < (NX - nx) * nsb; i += 256) xd[nx * nsb + i] = 0.f;
    } else if (NX * nsb * 4 <= 256) {
        // one record per thread: load, issue the weight prologue, then store
        const uint32_t i = tid < NX * nsb * 4 ? tid : 0;
        const uint32_t p = i / (nsb * 4), rem = i % (nsb * 4), sb = rem >> 2, cc = rem & 3;
        const uint32_t pp = p < nx ? p : 0;
        const uint8_t * xb = (const uint8_t *)col_pick<NX>(C.x, pp) + xqk_off(cols) + (size_t)sb * 292;
        u32x4 v[4];
        int bs[4];
        float dk;
        if constexpr (FMT == FMT_Q4_K) {
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
        dk = *(const float *)xb;
        prologue();
        issued = true;
        if (tid < NX * nsb * 4) {
            uint32_t * rec = (uint32_t *)(xr + (size_t)tid * XREC);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                rec[4 * k + 0] = v[k].x; rec[4 * k + 1] = v[k].y; rec[4 * k + 2] = v[k].z; rec[4 * k + 3] = v[k].w;
                rec[16 + k] = (uint32_t)bs[k];
            }
            if (cc == 0) xd[p * nsb + sb] = (p < nx) ? dk : 0.f;
        }
    } else {
        for (uint32_t i = tid; i < NX * nsb * 4; i += 256) {
            const uint32_t p = i / (nsb * 4), rem = i % (nsb * 4), sb = rem >> 2, cc = rem & 3;
            const uint32_t pp = p < nx ? p : 0;
            const uint8_t * xb = (const uint8_t *)col_pick<NX>(C.x, pp) + xqk_off(cols) + (size_t)sb * 292;
            uint32_t * rec = (uint32_t *)(xr + (size_t)i * XREC);
            int bs[4];
            if constexpr (FMT == FMT_Q4_K) {
                const uint32_t g0 = 2 * (cc >> 1), h = cc & 1;
                const uint32_t gs[4] = {g0, g0 + 1, g0 + 4, g0 + 5};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const u32x4 v = ld4(xb + 36 + 32 * gs[k] + 16 * h);
                    rec[4 * k + 0] = v.x; rec[4 * k + 1] = v.y; rec[4 * k + 2] = v.z; rec[4 * k + 3] = v.w;
                    bs[k] = *(const int16_t *)(xb + 4 + 2 * (2 * gs[k] + h));
                }
            } else {
                const uint32_t hh = cc >> 1, bb = cc & 1;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const u32x4 v = ld4(xb + 36 + 128 * hh + 32 * g + 16 * bb);
                    rec[4 * g + 0] = v.x; rec[4 * g + 1] = v.y; rec[4 * g + 2] = v.z; rec[4 * g + 3] = v.w;
                    bs[g] = 32 * (int)*(const int16_t *)(xb + 4 + 2 * (8 * hh + 2 * g + bb));
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) rec[16 + k] = (uint32_t)bs[k];
            if (cc == 0) xd[p * nsb + sb] = (p < nx) ? *(const float *)xb : 0.f;
        }
    }
    if (!issued) prologue();
    __syncthreads();

    // XREG (16 % nsb == 0): a lane's superblock position within a row is the
    // same for every chunk, so its activation record stays in registers.
    u32x4a xregs[NX][5];
    if constexpr (XREG) {
#pragma unroll
        for (int p = 0; p < NX; ++p)
#pragma unroll
            for (int k = 0; k < 5; ++k)
                xregs[p][k] = *(const u32x4a *)(xr + (((size_t)p * nsb + (s & (nsb - 1))) * 4 + c) * XREC + 16 * k);
    }
    const uint32_t magic = (uint32_t)((0x100000000ull + nsb - 1) / nsb);   // f / nsb, f < 2^16
    const uint32_t fk = tid & 3, fp = (tid >> 2) % NX, frl = tid / (4 * NX);
    uint32_t slot = 0;                                            // ring stage of the next chunk

    for (uint32_t bt = batch0; bt < nbatch; bt += G) {
        const uint32_t row0 = bt * nr;
        const uint32_t nrow = min(nr, rows - row0);
        const uint32_t nsbb = nrow * nsb;                       // superblocks in this batch
        const uint32_t nci = nci_of(bt);
        const uint8_t * wb = w + (size_t)row0 * rb;
        const bool fok = frl < nrow && fp < nx;
        float * const ycol = col_pick<NX>(C.y, fp);
        const float yold = ycol[row0 + (frl < nrow ? frl : nrow - 1)];
        for (uint32_t i = 0; i < nci; ++i) {
            // NI * (D - 1) loads were issued after this chunk's
            WAIT_VM(NI * (D - 1));
            uint8_t * st = myst + slot * WIN;
            const uint32_t f = (wave + 4 * i) * 16 + s;            // batch-local superblock
            const bool act = f < nsbb;
            const uint32_t ff = act ? f : nsbb - 1;
            const uint32_t rl = __umulhi(ff, magic);
            const uint32_t sb = ff - rl * nsb;
            const uint8_t * xrec = xr + ((size_t)sb * 4 + c) * XREC;
            int ia[NX], im[NX];
            uint32_t tag;
            if constexpr (FMT == FMT_Q4_K) {
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
                    int acc_i = 0, acc_m = 0;
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
                    acc_m = mn[0] * (int)bsv.x + mn[1] * (int)bsv.y + mn[2] * (int)bsv.z + mn[3] * (int)bsv.w;
                    ia[p] = acc_i;
                    im[p] = acc_m;
                }
            } else {
                const uint32_t so = (uint32_t)(((uintptr_t)(wb + (size_t)(wave + 4 * i) * 16 * B)) & 15u) + 210 * s;
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
            // all reads of this stage are done before it is refilled
            WAIT_LGKM0();
            issue_one(st);
            slot = slot + 1 == (uint32_t)D ? 0 : slot + 1;
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
        __syncthreads();
        {
            const uint32_t k = fk, p = fp, rl = frl;
            float acc = 0.f;
            if (fok) {
                const int * ti = TI + (rl * NX + p) * nsb;
                const int * tm = TM + (rl * NX + p) * nsb;
                const uint32_t * th = TH + rl * nsb;
                const float * xdp = xd + p * nsb;
                for (uint32_t sbi = k; sbi < nsb; sbi += 4) {
                    const float dk = xdp[sbi];
                    if constexpr (FMT == FMT_Q4_K) {
                        const float d = h2f(th[sbi] & 0xFFFFu), dmin = h2f(th[sbi] >> 16);
                        acc = fmaf(d * dk, (float)ti[sbi], acc);
                        acc = fmaf(-(dmin * dk), (float)tm[sbi], acc);
                    } else {
                        acc = fmaf(h2f(th[sbi]) * dk, (float)ti[sbi], acc);
                    }
                }
            }
            const float s01 = acc + qx1f(acc);
            const float r = s01 + qx2f(s01);
            if (fok && k == 0) ycol[row0 + rl] = yold + r;
        }
        __syncthreads();
    }
    // the trailing repeat loads still target this workgroup's LDS: drain them
    WAIT_VM(0);
}

template <int FMT, int NX, int D, bool FUSE, bool XREG>
__global__ __launch_bounds__(256) void k_dot_kstream(DotArgs a, uint32_t nr) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
    const uint8_t * w = a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0);
    KsCols<NX> C;
#pragma unroll
    for (int p = 0; p < NX; ++p) {
        const uint32_t pp = p < (int)a.nx ? p : 0;
        C.x[p] = a.x + (size_t)pp * a.xstride;
        C.y[p] = a.y + (size_t)pp * a.ystride;
    }
    ks_body<FMT, NX, D, FUSE, XREG>(w, a.rows, a.cols, C, a.nx, nr, blockIdx.x, gridDim.x, sm);
}

// Grouped expert matvec: blockIdx.y = expert.  The workgroup collects the
// routed (token, slot) pairs of its expert and streams that expert's weights
// once per group of NX pairs; with no pair routed to it, it exits before any
// weight byte is requested.
template <int FMT, int NX, int D, bool XREG>
__global__ __launch_bounds__(256) void k_moe_kstream(MoeArgs a, uint32_t nr) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
    __shared__ uint32_t pairs[256];
    __shared__ uint32_t npairs;
    const uint32_t e = blockIdx.y;
    if (threadIdx.x == 0) {
        uint32_t n = 0;
        for (uint32_t i = 0; i < a.ntok * a.top_k && n < 256; ++i)
            if (a.ids[i] == e) pairs[n++] = i;                    // i = tok * top_k + slot
        npairs = n;
    }
    __syncthreads();
    const uint32_t np = npairs;
    const uint8_t * w = a.w + (size_t)e * a.estride;
    for (uint32_t p0 = 0; p0 < np; p0 += NX) {
        const uint32_t nx = min((uint32_t)NX, np - p0);
        KsCols<NX> C;
#pragma unroll
        for (int p = 0; p < NX; ++p) {
            const uint32_t ts = pairs[p0 + ((uint32_t)p < nx ? p : 0)];
            const uint32_t xi = a.x_per_slot ? ts : ts / a.top_k;
            C.x[p] = a.x + (size_t)xi * a.xstride;
            C.y[p] = a.y + (size_t)ts * a.ystride;
        }
        ks_body<FMT, NX, D, false, XREG>(w, a.rows, a.cols, C, nx, nr, blockIdx.x, gridDim.x, sm);
        __syncthreads();
    }
}

// ----------------------------------------------------------------- launch --
struct KsTune { uint32_t wgs_per_cu, nr, D; };
static KsTune ks_tune() {
    static KsTune t = [] {
        KsTune d{2, 0, 0};
        if (const char * e = getenv("FLH_KS_TUNE")) {
            unsigned x = 0, y = 0, z = 0;
            if (sscanf(e, "%u,%u,%u", &x, &y, &z) == 3) d = KsTune{x, y, z};
        }
        return d;
    }();
    return t;
}

static size_t g_lds_limit = 0;
size_t lds_limit() {
    if (!g_lds_limit) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 65536;
        g_lds_limit = (size_t)v;
    }
    return g_lds_limit;
}

template <int FMT, int NX, int D, bool FUSE, bool XREG>
static int ks_launch_x(const DotArgs & a, uint32_t nr, uint32_t grid, size_t smb, hipStream_t s) {
    if (smb > 65536)
        (void)hipFuncSetAttribute((const void *)k_dot_kstream<FMT, NX, D, FUSE, XREG>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)smb);
    hipLaunchKernelGGL((k_dot_kstream<FMT, NX, D, FUSE, XREG>), dim3(grid), dim3(256), smb, s, a, nr);
    return hip_check(hipGetLastError(), "k_dot_kstream launch");
}
template <int FMT, int NX, int D, bool FUSE>
static int ks_launch_d(const DotArgs & a, uint32_t nr, uint32_t grid, size_t smb, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    if (16 % nsb == 0 && !getenv("FLH_NO_XREG")) return ks_launch_x<FMT, NX, D, FUSE, true>(a, nr, grid, smb, s);
    return ks_launch_x<FMT, NX, D, FUSE, false>(a, nr, grid, smb, s);
}

// Returns FLH_ERR_UNSUPPORTED (without launching) when the shape does not fit
// this kernel's LDS plan; the caller then uses the register-resident kernel.
// LDS plan: at most 64 KiB per workgroup (two workgroups per CU); shrink the
// batch first, then the ring depth; FLH_ERR_UNSUPPORTED if it cannot fit.
template <int FMT>
static int ks_plan(uint32_t rows, uint32_t nx_t, uint32_t nsb, uint32_t slots, int Ddef,
                   uint32_t & nr, int & D, size_t & smb) {
    const KsTune t = ks_tune();
    nr = t.nr ? t.nr : (rows + slots - 1) / slots;
    if (nr < 1) nr = 1;
    if (nr > 64u / nx_t) nr = 64u / nx_t;
    D = t.D ? (int)t.D : Ddef;
    const size_t lim = lds_limit() < 65536 ? lds_limit() : 65536;
    while (ks_smem_bytes<FMT>(nr, nx_t, nsb, D) > lim && nr > 4) nr >>= 1;
    while (ks_smem_bytes<FMT>(nr, nx_t, nsb, D) > lim && D > 2) --D;
    while (ks_smem_bytes<FMT>(nr, nx_t, nsb, D) > lim && nr > 1) nr >>= 1;
    smb = ks_smem_bytes<FMT>(nr, nx_t, nsb, D);
    return smb > lim ? FLH_ERR_UNSUPPORTED : FLH_OK;
}

template <int FMT, int NX, bool FUSE>
static int ks_launch(const DotArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    const KsTune t = ks_tune();
    const uint32_t slots = (uint32_t)num_cus() * (t.wgs_per_cu ? t.wgs_per_cu : 2);
    uint32_t nr;
    int D;
    size_t smb;
    if (ks_plan<FMT>(a.rows, NX, nsb, slots, FMT == FMT_Q4_K ? 4 : 3, nr, D, smb)) return FLH_ERR_UNSUPPORTED;
    const uint32_t nbatch = (a.rows + nr - 1) / nr;
    const uint32_t grid = nbatch < slots ? nbatch : slots;
    switch (D) {
        case 2: return ks_launch_d<FMT, NX, 2, FUSE>(a, nr, grid, smb, s);
        case 3: return ks_launch_d<FMT, NX, 3, FUSE>(a, nr, grid, smb, s);
        default: return ks_launch_d<FMT, NX, 4, FUSE>(a, nr, grid, smb, s);
    }
}

template <int FMT, int NX, int D, bool XREG>
static int moe_launch_x(const MoeArgs & a, uint32_t nr, uint32_t gx, size_t smb, hipStream_t s) {
    hipLaunchKernelGGL((k_moe_kstream<FMT, NX, D, XREG>), dim3(gx, a.n_expert), dim3(256), smb, s, a, nr);
    return hip_check(hipGetLastError(), "k_moe_kstream launch");
}
template <int FMT, int NX, int D>
static int moe_launch_d(const MoeArgs & a, uint32_t nr, uint32_t gx, size_t smb, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    if (16 % nsb == 0) return moe_launch_x<FMT, NX, D, true>(a, nr, gx, smb, s);
    return moe_launch_x<FMT, NX, D, false>(a, nr, gx, smb, s);
}
template <int FMT, int NX>
static int moe_launch(const MoeArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    // experts that can be active at once share the chip
    const uint32_t pairs = a.ntok * a.top_k;
    const uint32_t active = pairs < a.n_expert ? pairs : a.n_expert;
    const uint32_t gx = ((uint32_t)num_cus() * 2 + active - 1) / active;
    uint32_t nr;
    int D;
    size_t smb;
    if (ks_plan<FMT>(a.rows, NX, nsb, gx, FMT == FMT_Q4_K ? 4 : 3, nr, D, smb)) return FLH_ERR_UNSUPPORTED;
    const uint32_t nbatch = (a.rows + nr - 1) / nr;
    const uint32_t g = nbatch < gx ? nbatch : gx;
    switch (D) {
        case 2: return moe_launch_d<FMT, NX, 2>(a, nr, g, smb, s);
        case 3: return moe_launch_d<FMT, NX, 3>(a, nr, g, smb, s);
        default: return moe_launch_d<FMT, NX, 4>(a, nr, g, smb, s);
    }
}

int launch_moe_kstream(int fmt, const MoeArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    if (nsb == 0 || (a.cols & 255) || nsb > 64) return FLH_ERR_UNSUPPORTED;
    if ((uintptr_t)a.w & 15 || (a.estride & 15) || getenv("FLH_NO_KSTREAM")) return FLH_ERR_UNSUPPORTED;
    // columns per pass: the most pairs one expert can get, capped by what fits
    const uint32_t pairs = a.ntok * a.top_k;
    const uint32_t want = pairs < a.ntok ? pairs : a.ntok;     // an expert appears once per token
    int rc = FLH_ERR_UNSUPPORTED;
    if (fmt == FMT_Q4_K) {
        if (want >= 4) rc = moe_launch<FMT_Q4_K, 4>(a, s);
        if (rc == FLH_ERR_UNSUPPORTED && want >= 2) rc = moe_launch<FMT_Q4_K, 2>(a, s);
        if (rc == FLH_ERR_UNSUPPORTED) rc = moe_launch<FMT_Q4_K, 1>(a, s);
    } else if (fmt == FMT_Q6_K) {
        if (want >= 4) rc = moe_launch<FMT_Q6_K, 4>(a, s);
        if (rc == FLH_ERR_UNSUPPORTED && want >= 2) rc = moe_launch<FMT_Q6_K, 2>(a, s);
        if (rc == FLH_ERR_UNSUPPORTED) rc = moe_launch<FMT_Q6_K, 1>(a, s);
    }
    return rc;
}

template <bool FUSE>
static int ks_dispatch(int fmt, const DotArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    if (nsb == 0 || (a.cols & 255) || nsb > 64 || a.nx > 4) return FLH_ERR_UNSUPPORTED;
    if ((uintptr_t)a.w & 15 || (a.estride & 15)) return FLH_ERR_UNSUPPORTED;
    if (FUSE && (((uintptr_t)a.x & 15) || (a.xstride & 3))) return FLH_ERR_UNSUPPORTED;
    if (getenv("FLH_NO_KSTREAM")) return FLH_ERR_UNSUPPORTED;
    if (fmt == FMT_Q4_K)
        return a.nx == 1 ? ks_launch<FMT_Q4_K, 1, FUSE>(a, s) : a.nx == 2 ? ks_launch<FMT_Q4_K, 2, FUSE>(a, s)
                                                                         : ks_launch<FMT_Q4_K, 4, FUSE>(a, s);
    if (fmt == FMT_Q6_K)
        return a.nx == 1 ? ks_launch<FMT_Q6_K, 1, FUSE>(a, s) : a.nx == 2 ? ks_launch<FMT_Q6_K, 2, FUSE>(a, s)
                                                                         : ks_launch<FMT_Q6_K, 4, FUSE>(a, s);
    return FLH_ERR_UNSUPPORTED;
}

int launch_dot_kstream(int fmt, const DotArgs & a, hipStream_t s) { return ks_dispatch<false>(fmt, a, s); }
int launch_act_dot_kstream(int fmt, const DotArgs & a, hipStream_t s) { return ks_dispatch<true>(fmt, a, s); }

}  // namespace flh
