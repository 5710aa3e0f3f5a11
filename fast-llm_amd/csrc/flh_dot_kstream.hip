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
// (4 or 8 waves) owns a batch of nr whole rows; its chunks are dealt round-robin
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
#include "flh_kstream.h"
#include "flh_internal.h"
#include "flh_status.h"
#include <stdio.h>
#include <stdlib.h>
#include <atomic>
#include <mutex>
#include <unordered_map>

namespace flh {


// One pass over rows [0, rows) of the matrix at w for nx <= NX columns; the
// workgroup g of G owns the contiguous rows [rows*g/G, rows*(g+1)/G) (an
// even split: workgroups differ by at most one row), streamed in batches of at
// most nr rows.  Ends with every weight DMA
// drained, so the caller may start another pass on the same LDS.
template <int FMT, int NX, int D, bool FUSE, bool XREG, int KW = 4, bool NORM = false>
__device__ __forceinline__ void ks_body(const uint8_t * __restrict__ w, uint32_t rows, uint32_t cols,
                                        const KsCols<NX> & C, uint32_t nx, uint32_t nrp,
                                        uint32_t g, uint32_t G, uint8_t * sm, const NormArgs & nm = NormArgs{}) {
    // nrp: rows per batch | chunks issued by the prologue << 16 (0: D)
    const uint32_t nr = nrp & 0xFFFF;
    const uint32_t pro = (nrp >> 16) ? min(nrp >> 16, (uint32_t)D) : (uint32_t)D;
    constexpr uint32_t B = KS<FMT>::BLK, WIN = KS<FMT>::WIN;
    constexpr int NI = KS<FMT>::NI;
    const uint32_t nsb = cols >> 8;
    const uint64_t rb = (uint64_t)nsb * B;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    // wave-uniform: keeps the chunk cursor and batch logic on the scalar unit
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t s = lane >> 2, c = lane & 3;

    uint8_t * stages = sm;                                        // [4][D][WIN]
    uint8_t * xr = sm + (size_t)KW * D * WIN;                     // [NX][nsb][4][80]
    constexpr uint32_t TPS = ks_tps<FMT>();                      // fold terms per superblock
    float * xd = (float *)(xr + (size_t)NX * nsb * 4 * XREC);     // [NX][nsb * TPS]
    int * TI = (int *)(xd + (size_t)NX * nsb * TPS);              // [nr][NX][nsb * TPS]
    int * TM = TI + (size_t)nr * NX * nsb * TPS;                  // Q4_K only
    uint32_t * TH = (uint32_t *)(FMT == FMT_Q4_K ? TM + (size_t)nr * NX * nsb : TM);   // [nr][nsb * TPS]
    float * ysm = (float *)(TH + (size_t)nr * nsb * TPS);          // [64] old y of the batch
    uint8_t * myst = stages + (size_t)wave * D * WIN;

    KS_STAMP(0);
    const uint32_t rbeg = (uint32_t)((uint64_t)rows * g / G);
    const uint32_t rend = (uint32_t)((uint64_t)rows * (g + 1) / G);
    const uint32_t nbatch = (rend - rbeg + nr - 1) / nr;          // batches of this workgroup
    auto nci_of = [&](uint32_t bt) -> uint32_t {                  // this wave's chunks in batch bt
        const uint32_t nrow = min(nr, rend - rbeg - bt * nr);
        const uint32_t nch = (nrow * nsb + 15) / 16;
        return nch > wave ? (nch - wave + KW - 1) / KW : 0;
    };
    // Issue cursor over this wave's chunk sequence (batches blockIdx.x, +G, ...).
    // nissued counts the chunks whose DMA was issued; past the end of the
    // sequence nothing is issued, and the wait before each chunk counts only
    // the chunks really issued after it.
    uint32_t qbt = 0, qci = 0, qn = qbt < nbatch ? nci_of(qbt) : 0;
    uint32_t nissued = 0, ncons = 0;
    // Next chunk of the sequence: its batch's weight base, batch-local chunk
    // index and superblock count; false past the end.
    auto next_chunk = [&](const uint8_t *& base, uint32_t & ch, uint32_t & nsbb) -> bool {
        while (qbt < nbatch && qci >= qn) {
            ++qbt;
            qci = 0;
            qn = qbt < nbatch ? nci_of(qbt) : 0;
        }
        if (qbt >= nbatch) return false;
        base = w + (size_t)(rbeg + qbt * nr) * rb;
        ch = wave + KW * qci;
        nsbb = min(nr, rend - rbeg - qbt * nr) * nsb;
        return true;
    };
    auto issue_one = [&]() {
        const uint8_t * base;
        uint32_t ch, nsbb;
        if (next_chunk(base, ch, nsbb)) {
            ks_issue<FMT>(base, ch, nsbb, myst + (nissued % D) * WIN, lane);
            ++qci;
            ++nissued;
        }
    };
    // The first D chunks of the sequence are issued right after the
    // activation loads.  The first DMA is issued unconditionally (a wave with
    // no chunk re-reads the workgroup's first superblock into its idle stage),
    // so the compiler knows exactly NI loads follow the activation loads and
    // waits for the activation alone (vmcnt(NI)) instead of for the first
    // weight chunk as well.
    // Returns the number of chunk DMAs issued (the dummy counts: the caller
    // waits for the loads issued before them).
    auto prologue = [&]() -> uint32_t {
        const uint8_t * base = w + (size_t)rbeg * rb;
        uint32_t ch = 0, nsbb = 1;
        const bool real = next_chunk(base, ch, nsbb);
        ks_issue<FMT>(base, ch, nsbb, myst, lane);
        uint32_t n = 1;
        if (real) {
            ++qci;
            ++nissued;
#pragma unroll
            for (int j = 1; j < D; ++j) {
                if ((uint32_t)j < pro) {
                    const uint32_t before = nissued;
                    issue_one();
                    n += nissued - before;
                }
            }
        }
        return n;
    };

    // The batch's old y values (y += semantics) go to LDS by a DMA of wave 0:
    // a register load would make the compiler wait for every weight DMA in
    // flight before the fold.  The first batch's is issued before anything
    // else, later ones right after the previous fold; y_at = chunks issued
    // before it.
    uint32_t y_at = 0;
    auto issue_y = [&](uint32_t bt) {
        if (wave == 0 && bt < nbatch) {
            const uint32_t row0 = rbeg + bt * nr, nrow = min(nr, rend - row0);
            const uint32_t yr = lane / NX, yp = lane % NX;
            const bool yv = yr < nrow && yp < nx;
            const float * ya = yv ? col_pick<NX>(C.y, yp) + row0 + yr : C.y[0] + row0;
            __builtin_amdgcn_global_load_lds(GPTR(ya), LPTR(ysm), 4, 0, 0);
            y_at = nissued;
        }
    };
    issue_y(0);

    // ---- activation records, once per workgroup (overlaps the first weight DMAs)
    if constexpr (FUSE) ks_x_fuse<FMT, NX, NI, D, KW, NORM>(C, nx, nsb, cols, xr, xd, g, G, prologue, nm);
    else ks_x_app<FMT, NX, NI, D>(C, nx, nsb, cols, xr, xd, prologue);
    lds_barrier();
    KS_STAMP(1);

    // XREG (16 % nsb == 0): a lane's superblock position within a row is the
    // same for every chunk, so its activation record stays in registers.
    u32x4a xregs[NX][5];
    if constexpr (XREG) {
#pragma unroll
        for (int p = 0; p < NX; ++p) lds_ld_rec(xr + (((size_t)p * nsb + (s & (nsb - 1))) * 4 + c) * XREC, xregs[p]);
    }
    const uint32_t magic = div_magic(nsb);                        // f / nsb, f < 2^16
    const uint32_t fk = tid & 3, fp = (tid >> 2) % NX, frl = tid / (4 * NX);
    uint32_t slot = 0;                                            // ring stage of the next chunk

    for (uint32_t bt = 0; bt < nbatch; ++bt) {
        const uint32_t row0 = rbeg + bt * nr;
        const uint32_t nrow = min(nr, rend - row0);
        const uint32_t nsbb = nrow * nsb;                       // superblocks in this batch
        const uint32_t nci = nci_of(bt);
        const uint8_t * wb = w + (size_t)row0 * rb;
        const bool fok = frl < nrow && fp < nx;
        float * const ycol = col_pick<NX>(C.y, fp);
        if (bt != 0) issue_y(bt);
        for (uint32_t i = 0; i < nci; ++i) {
            // wait for this chunk's DMA: (nissued - 1 - ncons) chunks were issued after it
            ks_wait_behind<NI, D>(nissued - 1 - ncons);
            ++ncons;
            if (i == 0 && bt == 0) KS_STAMP(2);
            if (i == 1 && bt == 0) KS_STAMP(7);
            uint8_t * st = myst + slot * WIN;
            const uint32_t f = (wave + KW * i) * 16 + s;           // batch-local superblock
            const bool act = f < nsbb;
            const uint32_t ff = act ? f : nsbb - 1;
            const uint32_t rl = div_small(ff, magic);
            const uint32_t sb = ff - rl * nsb;
            int ia[NX], im[NX];
            uint32_t tag;
            const uint32_t mis = (uint32_t)(((uintptr_t)(wb + (size_t)(wave + KW * i) * 16 * B)) & 15u);
            ks_chunk<FMT, NX, XREG>(st, mis, s, c, xr + ((size_t)sb * 4 + c) * XREC, nsb, xregs, ia, im, tag);
            // all reads of this stage are done before it is refilled
            WAIT_LGKM0();
            // refill the ring to D chunks in flight (the prologue issued only pro)
            issue_one();
            if (ncons == 1)
                for (int j = 1; j < D; ++j)
                    if (nissued < ncons + D) issue_one();
            slot = slot + 1 == (uint32_t)D ? 0 : slot + 1;
            ks_park<FMT, NX>(ia, im, tag, act, c, nx, rl, sb, nsb, TI, TM, TH);
        }
        KS_STAMP(12);
        // wave 0: chunks issued after the y DMA are the only loads that can be
        // younger than it and still outstanding (at most D of them)
        if (wave == 0) ks_wait_behind<NI, D + 1>(min(nissued - y_at, (uint32_t)D));
        lds_barrier();
        KS_STAMP(3);
        const float r = ks_fold<FMT, NX>(TI, TM, TH, xd, nsb, fk, fp, frl, fok);
        KS_STAMP(8);
        if (fok && fk == 0) ycol[row0 + frl] = ysm[frl * NX + fp] + r;
        lds_barrier();
    }
    WAIT_VM(0);
    KS_STAMP(4);
}

template <int FMT, int NX, int D, bool FUSE, bool XREG, int KW = 4, bool NORM = false>
__global__ __launch_bounds__(64 * KW) void k_dot_kstream(DotArgs a, uint32_t nr, NormArgs nm) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
    const uint8_t * w = a.w + (a.id_slot ? (size_t)(*a.id_slot) * a.estride : 0);
    KsCols<NX> C;
#pragma unroll
    for (int p = 0; p < NX; ++p) {
        const uint32_t pp = p < (int)a.nx ? p : 0;
        C.x[p] = a.x + (size_t)pp * a.xstride;
        C.y[p] = a.y + (size_t)pp * a.ystride;
    }
    ks_body<FMT, NX, D, FUSE, XREG, KW, NORM>(w, a.rows, a.cols, C, a.nx, nr, blockIdx.x, gridDim.x, sm, nm);
}

// Grouped expert matvec: the routed experts share the grid (moe_assign).  The workgroup collects the
// routed (token, slot) pairs of its expert and streams that expert's weights
// once per group of NX pairs; with no pair routed to it, it exits before any
// weight byte is requested.
template <int FMT, int NX, int D, bool XREG>
__global__ __launch_bounds__(256) void k_moe_kstream(MoeArgs a, uint32_t nr) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
    __shared__ uint32_t pairs[256];
    __shared__ uint32_t rids[256];
    __shared__ uint32_t npairs;
    const uint32_t * ids = moe_route(a, rids);
    uint32_t g, G;
    const uint32_t e = moe_assign(ids, a.ntok * a.top_k, a.n_expert, blockIdx.y * gridDim.x + blockIdx.x,
                                  gridDim.x * gridDim.y, g, G);
    if (e >= a.n_expert) return;
    if (threadIdx.x == 0) {
        uint32_t n = 0;
        for (uint32_t i = 0; i < a.ntok * a.top_k && n < 256; ++i)
            if (ids[i] == e) pairs[n++] = i;                      // i = tok * top_k + slot
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
        ks_body<FMT, NX, D, false, XREG>(w, a.rows, a.cols, C, nx, nr, g, G, sm);
        __syncthreads();
    }
}

// ----------------------------------------------------------------- launch --
// Chunks each wave requests before the activation is staged (the rest of its
// ring is requested after its first chunk).  Reading a ready q8_K appendix
// takes about as long as the first chunk, and a smaller launch-time burst
// lands that chunk sooner: one (measured: Q4_K 4096x4096 5.6 -> 5.3 us).  A
// fused ACT_Q8 keeps the waves busy quantising well after the first chunk
// has landed: the whole ring (layer step 41.7 -> 40.3 us).
static uint32_t ks_pro(bool fuse) { return tune().ks_pro ? tune().ks_pro : fuse ? 2u : 1u; }

static std::atomic<size_t> g_lds_limit{0};
size_t lds_limit() {
    size_t l = g_lds_limit.load(std::memory_order_relaxed);
    if (!l) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 65536;
        l = (size_t)v;
        g_lds_limit.store(l, std::memory_order_relaxed);
    }
    return l;
}

// A kernel's static LDS (its __shared__ arrays), from the runtime, cached.
size_t static_lds(const void * kern) {
    static std::mutex mu;
    static std::unordered_map<const void *, size_t> cache;
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(kern);
    if (it != cache.end()) return it->second;
    hipFuncAttributes fa{};
    const size_t v = hipFuncGetAttributes(&fa, kern) == hipSuccess ? fa.sharedSizeBytes : 4096;
    (void)hipGetLastError();
    cache.emplace(kern, v);
    return v;
}

// Before a launch: the dynamic LDS of a plan plus the kernel's static LDS
// must fit one workgroup's LDS (a dispatch that asks for more is rejected by
// the device, and the queue with it).  FLH_ERR_UNSUPPORTED (the caller takes
// another kernel) otherwise.
int lds_fits(const void * kern, size_t dyn, const char * what) {
    if (dyn + static_lds(kern) <= lds_limit()) return FLH_OK;
    return set_error(FLH_ERR_UNSUPPORTED, what);
}

template <int FMT, int NX, int D, bool FUSE, bool XREG>
static int ks_launch_x(const DotArgs & a, uint32_t nr, uint32_t grid, size_t smb, hipStream_t s) {
    if (int rc = lds_fits((const void *)k_dot_kstream<FMT, NX, D, FUSE, XREG>, smb, "k_dot_kstream: LDS over the limit"))
        return rc;
    if (smb > 65536)
        (void)hipFuncSetAttribute((const void *)k_dot_kstream<FMT, NX, D, FUSE, XREG>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)smb);
    hipLaunchKernelGGL((k_dot_kstream<FMT, NX, D, FUSE, XREG>), dim3(grid), dim3(256), smb, s, a, nr | (ks_pro(FUSE) << 16),
                       NormArgs{});
    return hip_check(hipGetLastError(), "k_dot_kstream launch");
}
template <int FMT, int NX, int D, bool FUSE>
static int ks_launch_d(const DotArgs & a, uint32_t nr, uint32_t grid, size_t smb, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    if (16 % nsb == 0) return ks_launch_x<FMT, NX, D, FUSE, true>(a, nr, grid, smb, s);
    return ks_launch_x<FMT, NX, D, FUSE, false>(a, nr, grid, smb, s);
}

// Returns FLH_ERR_UNSUPPORTED (without launching) when the shape does not fit
// this kernel's LDS plan; the caller then uses the register-resident kernel.
// LDS plan: at most 64 KiB per workgroup (two workgroups per CU), or `capv`
// when given (one workgroup per CU: several columns of wide rows, whose
// activation records alone take 36-73 KB); shrink the batch first, then the
// ring depth; FLH_ERR_UNSUPPORTED if it cannot fit.
template <int FMT>
static int ks_plan(uint32_t rows, uint32_t nx_t, uint32_t nsb, uint32_t slots, int Ddef,
                   uint32_t & nr, int & D, size_t & smb, int KW = 4, size_t capv = 0) {
    const Tune & t = tune();
    nr = t.ks_nr ? t.ks_nr : (rows + slots - 1) / slots;
    if (nr < 1) nr = 1;
    if (nr > 64u / nx_t) nr = 64u / nx_t;
    D = t.ks_D ? (int)t.ks_D : Ddef;
    const size_t cap = capv ? capv : KW == 4 ? 65536 : 81920;      // two workgroups per CU / one
    const size_t lim = lds_limit() < cap ? lds_limit() : cap;
    while (ks_smem_bytes<FMT>(nr, nx_t, nsb, D, KW) > lim && nr > 4) nr >>= 1;
    while (ks_smem_bytes<FMT>(nr, nx_t, nsb, D, KW) > lim && D > 2) --D;
    while (ks_smem_bytes<FMT>(nr, nx_t, nsb, D, KW) > lim && nr > 1) nr >>= 1;
    // equal batches: a workgroup's ceil(rows / slots) rows in the fewest batches
    const uint32_t g = rows < slots ? rows : slots;
    const uint32_t rpw = (rows + g - 1) / g, nb = (rpw + nr - 1) / nr;
    nr = (rpw + nb - 1) / nb;
    smb = ks_smem_bytes<FMT>(nr, nx_t, nsb, D, KW);
    return smb > lim ? FLH_ERR_UNSUPPORTED : FLH_OK;
}

template <int FMT, int NX, bool FUSE>
static int ks_launch(const DotArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    const Tune & t = tune();
    if ((FMT == FMT_Q4_K || ((FMT == FMT_Q8_0 || FMT == FMT_Q6_K) && !FUSE)) && NX == 1 && t.sbl) {
        const int rc = launch_dot_sbl(FMT, a, FUSE, s);
        if (rc != FLH_ERR_UNSUPPORTED) return rc;
    }
    if constexpr (NX == 1) {
        // Two 8-wave workgroups per CU (16 waves) for single-column dots with
        // a fused ACT_Q8 or more than 16 superblocks per row: measured, the
        // Llama-3-8B layer step 41.8 -> 40.6 us (down 4096x14336 9.9 -> 9.2,
        // the fused ops each a little); the unfused 4096-column shapes stay on
        // 4-wave workgroups (O 4096x4096: 5.2 vs 5.4 us).  Tune::ks_w8_*
        // overrides.
        const unsigned w8a = t.ks_w8_mode, w8b = t.ks_w8_wgs;
        const unsigned bit = (FUSE ? 1u : 4u) << (nsb > 16 ? 0 : 1);
        const bool use = (w8a & bit) != 0;
        if (use) {
            const uint32_t slots = (uint32_t)num_cus() * (w8b ? w8b : 1);
            uint32_t nr;
            int D;
            size_t smb;
            if (ks_plan<FMT>(a.rows, 1, nsb, slots, 2, nr, D, smb, 8) == FLH_OK && D == 2) {
                const uint32_t grid = a.rows < slots ? a.rows : slots;
                auto go = [&](auto kern) {
                    if (int rc = lds_fits((const void *)kern, smb, "k_dot_kstream: LDS over the limit")) return rc;
                    (void)hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smb);
                    hipLaunchKernelGGL(kern, dim3(grid), dim3(512), smb, s, a, nr | (ks_pro(FUSE) << 16), NormArgs{});
                    return hip_check(hipGetLastError(), "k_dot_kstream launch");
                };
                if (16 % nsb == 0) return go(k_dot_kstream<FMT, 1, 2, FUSE, true, 8>);
                return go(k_dot_kstream<FMT, 1, 2, FUSE, false, 8>);
            }
        }
    }
    uint32_t slots = (uint32_t)num_cus() * (t.ks_wgs_per_cu ? t.ks_wgs_per_cu : 2);
    uint32_t nr;
    int D;
    size_t smb;
    if (ks_plan<FMT>(a.rows, NX, nsb, slots, 2, nr, D, smb)) {
        // several columns of wide rows: one workgroup per CU (Q6_K 4096x14336,
        // 2 / 4 columns: 30.2 / 33.5 us on the register kernel)
        slots = (uint32_t)num_cus();
        if (NX == 1 || ks_plan<FMT>(a.rows, NX, nsb, slots, 2, nr, D, smb, 4, lds_limit()))
            return FLH_ERR_UNSUPPORTED;
    }
    const uint32_t grid = a.rows < slots ? a.rows : slots;
    switch (D) {
        case 2: return ks_launch_d<FMT, NX, 2, FUSE>(a, nr, grid, smb, s);
        case 3: return ks_launch_d<FMT, NX, 3, FUSE>(a, nr, grid, smb, s);
        default: return ks_launch_d<FMT, NX, 4, FUSE>(a, nr, grid, smb, s);
    }
}

template <int FMT, int NX, int D, bool XREG>
static int moe_launch_x(const MoeArgs & a, uint32_t nr, uint32_t gx, size_t smb, hipStream_t s) {
    if (moe_rows(a) == 0) return FLH_OK;
    if (int rc = lds_fits((const void *)k_moe_kstream<FMT, NX, D, XREG>, smb, "k_moe_kstream: LDS over the limit"))
        return rc;
    if (smb > 65536)
        (void)hipFuncSetAttribute((const void *)k_moe_kstream<FMT, NX, D, XREG>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)smb);
    hipLaunchKernelGGL((k_moe_kstream<FMT, NX, D, XREG>), dim3(gx, moe_rows(a)), dim3(256), smb, s, a, nr | (ks_pro(false) << 16));
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
    uint32_t gx = ((uint32_t)num_cus() * 2 + active - 1) / active;
    uint32_t nr;
    int D;
    size_t smb;
    if (ks_plan<FMT>(a.rows, NX, nsb, gx, 2, nr, D, smb)) {
        gx = ((uint32_t)num_cus() + active - 1) / active;        // one workgroup per CU
        if (NX == 1 || ks_plan<FMT>(a.rows, NX, nsb, gx, 2, nr, D, smb, 4, lds_limit())) return FLH_ERR_UNSUPPORTED;
    }
    const uint32_t g = a.rows < gx ? a.rows : gx;
    switch (D) {
        case 2: return moe_launch_d<FMT, NX, 2>(a, nr, g, smb, s);
        case 3: return moe_launch_d<FMT, NX, 3>(a, nr, g, smb, s);
        default: return moe_launch_d<FMT, NX, 4>(a, nr, g, smb, s);
    }
}

// RMSNORM -> ACT_Q8 -> Q4_K one-column dot on this kernel: 8-wave
// workgroups (the plan of its fused single-column launches), at most 8
// superblocks per wave (<= 16384 columns); FLH_ERR_UNSUPPORTED (nothing
// launched) when the plan does not fit.
int launch_norm_dot_kstream(const DotArgs & a, const NormArgs & nm, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    if (nsb == 0 || (a.cols & 255) || nsb > 64 || a.nx != 1 || ((uintptr_t)a.w & 15) || (a.estride & 15) ||
        ((uintptr_t)a.x & 15) || ((uintptr_t)nm.x & 15) || ((uintptr_t)nm.wn & 15))
        return FLH_ERR_UNSUPPORTED;
    const Tune & t = tune();
    const uint32_t slots = (uint32_t)num_cus() * (t.ks_w8_wgs ? t.ks_w8_wgs : 1);
    uint32_t nr;
    int D;
    size_t smb;
    if (ks_plan<FMT_Q4_K>(a.rows, 1, nsb, slots, 2, nr, D, smb, 8) != FLH_OK || D != 2) return FLH_ERR_UNSUPPORTED;
    const uint32_t grid = a.rows < slots ? a.rows : slots;
    auto go = [&](auto kern) {
        if (int rc = lds_fits((const void *)kern, smb, "k_dot_kstream: LDS over the limit")) return rc;
        (void)hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smb);
        hipLaunchKernelGGL(kern, dim3(grid), dim3(512), smb, s, a, nr | (ks_pro(true) << 16), nm);
        return hip_check(hipGetLastError(), "k_dot_kstream launch");
    };
    if (16 % nsb == 0) return go(k_dot_kstream<FMT_Q4_K, 1, 2, true, true, 8, true>);
    return go(k_dot_kstream<FMT_Q4_K, 1, 2, true, false, 8, true>);
}

int launch_moe_kstream(int fmt, const MoeArgs & a, hipStream_t s) {
    const uint32_t nsb = a.cols >> 8;
    if (nsb == 0 || (a.cols & 255) || nsb > 64) return FLH_ERR_UNSUPPORTED;
    if ((uintptr_t)a.w & 15 || (a.estride & 15)) return FLH_ERR_UNSUPPORTED;
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
    if (nsb == 0 || (a.cols & 255) || nsb > 64 || a.nx > (FUSE ? 4u : 8u)) return FLH_ERR_UNSUPPORTED;
    if ((uintptr_t)a.w & 15 || (a.estride & 15)) return FLH_ERR_UNSUPPORTED;
    if (FUSE && (((uintptr_t)a.x & 15) || (a.xstride & 3))) return FLH_ERR_UNSUPPORTED;
    if (fmt == FMT_Q4_K)
        return a.nx == 1 ? ks_launch<FMT_Q4_K, 1, FUSE>(a, s) : a.nx == 2 ? ks_launch<FMT_Q4_K, 2, FUSE>(a, s)
                                                                         : ks_launch<FMT_Q4_K, 4, FUSE>(a, s);
    if (fmt == FMT_Q6_K) {
        if constexpr (!FUSE)       // 5-8 columns in one pass (Q6_K below the matrix-core kernel's row floor)
            if (a.nx > 4) return ks_launch<FMT_Q6_K, 8, false>(a, s);
        return a.nx == 1 ? ks_launch<FMT_Q6_K, 1, FUSE>(a, s) : a.nx == 2 ? ks_launch<FMT_Q6_K, 2, FUSE>(a, s)
                                                                         : ks_launch<FMT_Q6_K, 4, FUSE>(a, s);
    }
    if (a.nx > 4) return FLH_ERR_UNSUPPORTED;
    if constexpr (!FUSE) {                    // Q8_0 x q8_1 (ACT_Q8 runs separately)
        if (fmt == FMT_Q8_0)
            return a.nx == 1 ? ks_launch<FMT_Q8_0, 1, false>(a, s) : a.nx == 2 ? ks_launch<FMT_Q8_0, 2, false>(a, s)
                                                                             : ks_launch<FMT_Q8_0, 4, false>(a, s);
    }
    return FLH_ERR_UNSUPPORTED;
}

#ifdef FLH_TRACE
extern "C" int flh_ks_trace(uint64_t * host, size_t n) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_ks_trace), n * 8, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -2;
}
#endif

int launch_dot_kstream(int fmt, const DotArgs & a, hipStream_t s) { return ks_dispatch<false>(fmt, a, s); }
int launch_act_dot_kstream(int fmt, const DotArgs & a, hipStream_t s) { return ks_dispatch<true>(fmt, a, s); }

}  // namespace flh
