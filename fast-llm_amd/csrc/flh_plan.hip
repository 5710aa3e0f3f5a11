// flh_plan.hip -- persistent executor for a frozen task table (one launch per
// token step instead of one per task).
//
// The reference runs its frozen task graph with a persistent GPU kernel that
// pops ready tiles from queues in unified memory
// (src/runtime/gpu_exec.cu:156-344; dependency counts dep_init/dep_count,
// fastllm.h:65-97).  Here the table is compiled on the host into OPS (a
// matrix's fused row tiles, an ACT_Q8, a SILU_MUL[+ACT_Q8]) with producer
// sets, each op split into ITEMS.  One workgroup per resident slot walks the
// items blockIdx.x, blockIdx.x + G, ... in index order (ops are in
// topological order, so an item only ever waits for items with smaller
// indices, all held by co-resident workgroups: no deadlock).
//
// What this buys over one launch per op: each wave's weight cursor runs
// ahead across item and op boundaries.  The weights of the next op never
// depend on the previous op's output, so their direct-to-LDS loads are in
// flight while the workgroup waits for its activation; only the activation
// reads wait.  The per-launch start-up and drain (~4 us on MI355X) is paid
// once per plan.
//
// Synchronisation: an item's outputs are written by wave 0 (DOT) or by all
// waves (ACT), released at agent scope, then counted with an agent-scope
// atomic add on the op's done counter.  A consumer's thread 0 polls the
// counters of the producers it has not seen complete, then every wave
// acquires at agent scope before reading the activation (the L2s of the
// XCDs are not coherent with each other for ordinary loads).  Waits are
// bounded: past spin_limit polls the error flag is set and the item runs
// anyway, so every wave always exits.  The last workgroup to finish resets
// the counters, so the next launch (or graph replay) starts from zero.
#include "flh_kstream.h"
#include "flh_internal.h"
#include "flh_status.h"

namespace flh {

template <int FMT> __host__ __device__ constexpr int plan_depth() { return FMT == FMT_Q4_K ? 4 : 3; }

template <bool XRG> struct BoolC { static constexpr bool value = XRG; };

#ifndef FLH_PLAN_ACQ
#define FLH_PLAN_ACQ 1
#endif
#ifndef FLH_PLAN_REL
#define FLH_PLAN_REL 1
#endif
// Diagnostic builds (-DFLH_PLAN_TRACE) record, per workgroup and item, the
// 100 MHz real-time clock at: item start, producers seen, activation ready,
// wave 0's chunk loop done, item signalled.
#ifdef FLH_PLAN_TRACE
#define PTRACE(j, k) do { if (pa.trace && tid == 0 && (j) < 8) \
    pa.trace[((size_t)blockIdx.x * 8 + (j)) * 6 + (k)] = __builtin_amdgcn_s_memrealtime(); } while (0)
#define PTRACE_OP(j, op) do { if (pa.trace && tid == 0 && (j) < 8) \
    pa.trace[((size_t)blockIdx.x * 8 + (j)) * 6 + 5] = (op); } while (0)
#else
#define PTRACE(j, k) do { } while (0)
#define PTRACE_OP(j, op) do { } while (0)
#endif

__device__ __forceinline__ void plan_acquire() {
#if FLH_PLAN_ACQ
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#endif
}
__device__ __forceinline__ void plan_release() {
#if FLH_PLAN_REL
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
#else
    __builtin_amdgcn_s_waitcnt(0);
#endif
}

template <int FMT>
__global__ __launch_bounds__(256) void k_plan(PlanArgs pa) {
    constexpr uint32_t B = KS<FMT>::BLK, WIN = KS<FMT>::WIN;
    constexpr int NI = KS<FMT>::NI, D = plan_depth<FMT>();
    extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
    __shared__ float yres[64];
    // the op table is read-only for the whole launch: constant address space,
    // so its (wave-uniform) reads are scalar loads
    const __attribute__((address_space(4))) PlanOp * ops =
        (const __attribute__((address_space(4))) PlanOp *)pa.ops;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t s = lane >> 2, c = lane & 3;
    const uint32_t G = gridDim.x, nops = pa.nops, nitems = pa.nitems;
    uint8_t * myst = sm + (size_t)wave * D * WIN;
    uint8_t * xr = sm + (size_t)4 * D * WIN;
    int * TI = (int *)(sm + pa.term_off);

    // ---- weight cursor: this wave's chunks of the workgroup's DOT items, in order.
    // Every issue is exactly NI loads (a repeat of a valid address once the
    // sequence is exhausted), so NI * (D - 1) loads always follow a chunk's.
    uint32_t cj = 0, cop = 0, qci = 0, qn = 0;
    bool cend = false;
    auto cur_load = [&]() {
        cj = __builtin_amdgcn_readfirstlane(cj);
        cop = __builtin_amdgcn_readfirstlane(cop);
        const uint32_t it = blockIdx.x + cj * G;
        if (it >= nitems) {
            cend = true;
            qn = 0;
            return;
        }
        while (cop + 1 < nops && it >= ops[cop + 1].item0) ++cop;
        if (ops[cop].kind != PLOP_DOT) {
            qn = 0;
            return;
        }
        const uint32_t nsb = ops[cop].cols >> 8, b = it - ops[cop].item0;
        const uint32_t nrow = min(ops[cop].nr, ops[cop].rows - b * ops[cop].nr);
        const uint32_t nch = (nrow * nsb + 15) / 16;
        qn = nch > wave ? (nch - wave + 3) / 4 : 0;
    };
    cur_load();
    const uint8_t * l_wb = pa.wdummy;
    uint32_t l_ch = 0, l_nsbb = 1;
    auto issue_one = [&](uint8_t * stage) {
        while (!cend && qci >= qn) {
            ++cj;
            qci = 0;
            cur_load();
        }
        if (!cend) {
            cop = __builtin_amdgcn_readfirstlane(cop);
            const uint32_t nsb = ops[cop].cols >> 8, b = blockIdx.x + cj * G - ops[cop].item0;
            const uint32_t nrow = min(ops[cop].nr, ops[cop].rows - b * ops[cop].nr);
            l_wb = ops[cop].w + (size_t)b * ops[cop].nr * nsb * B;
            l_ch = wave + 4 * qci;
            l_nsbb = nrow * nsb;
            ++qci;
        }
        ks_issue<FMT>(l_wb, l_ch, l_nsbb, stage, lane);
    };
    bool primed = false;
    auto prologue = [&]() {
        if (primed) return;
        primed = true;
#pragma unroll
        for (int j = 0; j < D; ++j) issue_one(myst + j * WIN);
    };

    // ---- producer waits
    uint32_t seen = 0;                          // ops known complete (workgroup-uniform)
    auto wait_for = [&](uint32_t prod) {
        const uint32_t need = prod & ~seen;
        if (!need) return;
        if (tid == 0) {
            uint32_t m = need;
            while (m) {
                const uint32_t k = __builtin_ctz(m);
                m &= m - 1;
                const uint32_t target = ops[k].nitems;
                uint32_t n = 0;
                while (__hip_atomic_load(&pa.ctl[2 + k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
                    if (++n > pa.spin_limit) {
                        __hip_atomic_store(&pa.ctl[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
        }
        __syncthreads();
        plan_acquire();
        seen |= need;
    };

    int xop = -1;                               // op whose activation records are in LDS
    uint32_t slot = 0, mop = 0;
    for (uint32_t j = 0;; ++j) {
        const uint32_t it = blockIdx.x + j * G;
        if (it >= nitems) break;
        while (mop + 1 < nops && it >= ops[mop + 1].item0) ++mop;
        mop = __builtin_amdgcn_readfirstlane(mop);
        const uint32_t b = it - ops[mop].item0;
        const uint32_t kind = ops[mop].kind, flags = ops[mop].flags, cols = ops[mop].cols;
        PTRACE(j, 0);
        PTRACE_OP(j, mop);

        if (kind == PLOP_ACT) {
            // SILU_MUL (h = silu(g) * u, src/runtime/decode_params.h:267-272)
            // and/or ACT_Q8 of one 256-element chunk per wave
            prologue();
            wait_for(ops[mop].prod);
            PTRACE(j, 1);
            const uint32_t nch = cols >> 8, nr = ops[mop].nr;
            const uint32_t ce = min((b + 1) * nr, nch);
            for (uint32_t ch = b * nr + wave; ch < ce; ch += 4) {
                const uint32_t e0 = ch * 256 + lane * 4;
                float v[4];
                if (flags & PLF_SILU) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float g = ops[mop].x[e0 + q];
                        v[q] = (g / (1.0f + expf(-g))) * ops[mop].u[e0 + q];
                        ops[mop].y[e0 + q] = v[q];
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] = ops[mop].y[e0 + q];
                }
                if (!(flags & PLF_NOQ)) {
                    uint8_t * yb = (uint8_t *)ops[mop].y;
                    act_q8_lanes(v, lane, ch, yb + xq_off(cols), yb + xqk_off(cols), cols);
                }
            }
            plan_release();
            __syncthreads();
            if (tid == 0) __hip_atomic_fetch_add(&pa.ctl[2 + mop], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            PTRACE(j, 4);
            continue;
        }

        // ---- DOT item: rows [row0, row0 + nrow) of the op's matrix
        const uint32_t nsb = cols >> 8, nr = ops[mop].nr;
        const uint32_t row0 = b * nr, nrow = min(nr, ops[mop].rows - row0);
        float * xd = (float *)(xr + (size_t)nsb * 4 * XREC);
        int * TM = TI + (size_t)nr * nsb;
        uint32_t * TH = (uint32_t *)(FMT == FMT_Q4_K ? TM + (size_t)nr * nsb : TM);
        float * y = ops[mop].y;
        if ((int)mop != xop) {
            wait_for(ops[mop].prod);
            PTRACE(j, 1);
            KsCols<1> C;
            C.x[0] = ops[mop].x;
            C.y[0] = y;
            if (flags & PLF_FUSE) ks_x_fuse<FMT, 1>(C, 1, nsb, cols, xr, xd, b == 0, prologue);
            else ks_x_app<FMT, 1>(C, 1, nsb, cols, xr, xd, prologue);
            __syncthreads();
            xop = (int)mop;
        }
        prologue();
        PTRACE(j, 2);
        float yold = 0.f;
        if (wave == 0 && lane < nrow) yold = y[row0 + lane];

        const uint32_t magic = (uint32_t)((0x100000000ull + nsb - 1) / nsb);   // f / nsb, f < 2^16
        const uint32_t nsbb = nrow * nsb;
        const uint32_t nch = (nsbb + 15) / 16;
        const uint32_t nci = nch > wave ? (nch - wave + 3) / 4 : 0;
        const uint8_t * wb = ops[mop].w + (size_t)row0 * nsb * B;
        u32x4a xregs[1][5];
        auto run = [&](auto XR) {
            constexpr bool XRG = decltype(XR)::value;
            if constexpr (XRG) {
#pragma unroll
                for (int k = 0; k < 5; ++k)
                    xregs[0][k] = *(const u32x4a *)(xr + ((size_t)(s & (nsb - 1)) * 4 + c) * XREC + 16 * k);
            }
            for (uint32_t i = 0; i < nci; ++i) {
                WAIT_VM(NI * (D - 1));
                uint8_t * st = myst + slot * WIN;
                const uint32_t f = (wave + 4 * i) * 16 + s;        // item-local superblock
                const bool act = f < nsbb;
                const uint32_t ff = act ? f : nsbb - 1;
                const uint32_t rl = __umulhi(ff, magic);
                const uint32_t sb = ff - rl * nsb;
                int ia[1], im[1];
                uint32_t tag;
                const uint32_t mis = (uint32_t)(((uintptr_t)(wb + (size_t)(wave + 4 * i) * 16 * B)) & 15u);
                ks_chunk<FMT, 1, XRG>(st, mis, s, c, xr + ((size_t)sb * 4 + c) * XREC, nsb, xregs, ia, im, tag);
                WAIT_LGKM0();                                      // stage read before its refill
                issue_one(st);
                slot = slot + 1 == (uint32_t)D ? 0 : slot + 1;
                ks_park<FMT, 1>(ia, im, tag, act, c, 1, rl, sb, nsb, TI, TM, TH);
            }
        };
        if (flags & PLF_XREG) run(BoolC<true>{});
        else run(BoolC<false>{});
        PTRACE(j, 3);
        __syncthreads();
        {
            const uint32_t fk = tid & 3, frl = tid >> 2;
            const float r = ks_fold<FMT, 1>(TI, TM, TH, xd, nsb, fk, 0, frl, frl < nrow);
            if (frl < nrow && fk == 0) yres[frl] = r;
        }
        __syncthreads();
        if (wave == 0) {
            if (lane < nrow) y[row0 + lane] = yold + yres[lane];
            plan_release();
            if (lane == 0) __hip_atomic_fetch_add(&pa.ctl[2 + mop], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        PTRACE(j, 4);
    }
    prologue();                                 // a workgroup without items still balances its loads
    __syncthreads();
    if (tid == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const uint32_t old = __hip_atomic_fetch_add(&pa.ctl[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == G - 1) {                     // every other workgroup is past its last wait
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            for (uint32_t k = 0; k < nops; ++k)
                __hip_atomic_store(&pa.ctl[2 + k], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&pa.ctl[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // trailing repeat loads still target this workgroup's LDS: drain them
    WAIT_VM(0);
}

size_t plan_stage_bytes(int fmt) {
    return fmt == FMT_Q4_K ? (size_t)4 * plan_depth<FMT_Q4_K>() * KS<FMT_Q4_K>::WIN
                           : (size_t)4 * plan_depth<FMT_Q6_K>() * KS<FMT_Q6_K>::WIN;
}

static const void * plan_fn(int fmt) {
    return fmt == FMT_Q4_K ? (const void *)k_plan<FMT_Q4_K> : (const void *)k_plan<FMT_Q6_K>;
}

int plan_occupancy(int fmt, size_t smb, int * blocks_per_cu) {
    const void * f = plan_fn(fmt);
    if (smb > 65536)
        if (int rc = hip_check(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smb),
                               "hipFuncSetAttribute(k_plan)")) return rc;
    return hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, f, 256, smb),
                     "hipOccupancyMaxActiveBlocksPerMultiprocessor(k_plan)");
}

int launch_plan(int fmt, const PlanArgs & a, uint32_t grid, size_t smb, hipStream_t s) {
    if (fmt == FMT_Q4_K) hipLaunchKernelGGL(k_plan<FMT_Q4_K>, dim3(grid), dim3(256), smb, s, a);
    else hipLaunchKernelGGL(k_plan<FMT_Q6_K>, dim3(grid), dim3(256), smb, s, a);
    return hip_check(hipGetLastError(), "k_plan launch");
}

}  // namespace flh
