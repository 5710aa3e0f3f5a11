// flh_common.h -- device helpers shared by the gfx950 kernels.
//
// Everything here is exact integer / bit work, or a single IEEE operation,
// so kernels built on it reproduce the reference CPU path bit for bit when
// the translation units are compiled with -ffp-contract=off.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>
#include "flh_iq_grids.h"

namespace flh {

// Fmt numeric values (reference include/fastllm/fastllm.h:56-57).
enum : int { FMT_F32 = 0, FMT_Q8_0 = 1, FMT_Q5_0 = 2, FMT_Q4_K = 3, FMT_Q6_K = 4,
             FMT_IQ2_XXS = 5, FMT_IQ3_XXS = 6 };

// Activation appendix offsets of one column (reference
// src/runtime/quants.h:302-330): [f32 x cols][pad16][q8_1 x cols/32][pad16]
// [q8_K x cols/256].  q8_1 = {f16 d, f16 s, i8 qs[32]} (36 B); q8_K =
// {f32 d, i16 bsums[16], i8 qs[256]} (292 B).
__host__ __device__ inline size_t xq_off(uint32_t cols) {
    return ((size_t)cols * 4 + 15) & ~(size_t)15;
}
__host__ __device__ inline size_t xqk_off(uint32_t cols) {
    return xq_off(cols) + ((((size_t)cols / 32) * 36 + 15) & ~(size_t)15);
}
__host__ __device__ inline size_t x_alloc_bytes(uint32_t cols) {
    return xqk_off(cols) + ((size_t)cols / 256) * 292;
}

// binary16 -> binary32.  v_cvt_f32_f16 is exact for every finite half
// (f16 denormals are preserved in the default HIP float mode).
__device__ __forceinline__ float h2f(uint32_t h16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

// binary32 -> binary16, round to nearest even, NaN -> 0x7E00|sign; the same
// mapping as the reference's fl_float2half (src/runtime/quants.h:333-356),
// written from the IEEE definition.
__device__ __forceinline__ uint32_t f2h(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a >= 0x47800000u) return sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u);
    if (a < 0x38800000u) {
        const uint32_t e = a >> 23;
        if (e < 102u) return sign;
        const uint32_t m = (a & 0x7FFFFFu) | 0x800000u, sh = 126u - e;
        uint32_t q = m >> sh;
        const uint32_t r = m & ((1u << sh) - 1u), hb = 1u << (sh - 1u);
        if (r > hb || (r == hb && (q & 1u))) ++q;
        return sign | q;
    }
    uint32_t q = (((a >> 23) - 112u) << 10) | ((a >> 13) & 0x3FFu);
    const uint32_t r = a & 0x1FFFu;
    if (r > 0x1000u || (r == 0x1000u && (q & 1u))) ++q;
    return sign | q;
}

// 4 x int8 dot product accumulate (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// ({hi,lo} >> 8*sh)[31:0], sh in 0..3 (v_alignbyte_b32).
__device__ __forceinline__ uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t sh) {
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
}

// floor(i / n) by multiply-high, exact for i < 2^16 and 1 <= n < 2^16:
// m = div_magic(n) = ceil(2^32 / n), which does not fit 32 bits for n == 1
// (stored as 0: the quotient is i itself).
__host__ __device__ inline uint32_t div_magic(uint32_t n) { return (uint32_t)((0x100000000ull + n - 1) / n); }
__device__ __forceinline__ uint32_t div_small(uint32_t i, uint32_t m) { return m ? __umulhi(i, m) : i; }

// DPP quad permutations: exchange with lane^1 / lane^2 inside each quad.
__device__ __forceinline__ int qx1(int v) {
    return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);   // [1,0,3,2]
}
__device__ __forceinline__ int qx2(int v) {
    return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);   // [2,3,0,1]
}
__device__ __forceinline__ float qx1f(float v) { return __int_as_float(qx1(__float_as_int(v))); }
__device__ __forceinline__ float qx2f(float v) { return __int_as_float(qx2(__float_as_int(v))); }
// The value of lane ^ o (o = 1, 2, 4, 8, 16, 32) in the calling lane: the data
// __shfl_xor(v, o) returns, moved by DPP (quad permutations, row shifts by 4,
// row rotation by 8) and the gfx950 permlane swaps (rows of 16, halves of
// 32) instead of an LDS permute.  o must be a compile-time constant.
__device__ __forceinline__ float xor_lane(float v, int o, uint32_t lane) {
    const int x = __float_as_int(v);
    if (o == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
    if (o == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
    if (o == 4) {
        const int l4 = __builtin_amdgcn_mov_dpp(x, 0x104, 0xF, 0xF, false);   // row_shl:4 (lane + 4)
        const int r4 = __builtin_amdgcn_mov_dpp(x, 0x114, 0xF, 0xF, false);   // row_shr:4 (lane - 4)
        return __int_as_float((lane & 4) ? r4 : l4);
    }
    if (o == 8) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false));   // row_ror:8
    if (o == 16) {
        // odd rows of the first operand <-> even rows of the second
        const auto sw = __builtin_amdgcn_permlane16_swap((uint32_t)x, (uint32_t)x, false, false);
        return __uint_as_float((lane & 16) ? sw[0] : sw[1]);
    }
    // upper half of the first operand <-> lower half of the second
    const auto sw = __builtin_amdgcn_permlane32_swap((uint32_t)x, (uint32_t)x, false, false);
    return __uint_as_float((lane & 32) ? sw[0] : sw[1]);
}

// DPP row mirrors: lane i <- lane 7-i inside each 8-lane half row, and lane
// i <- lane 15-i inside each 16-lane row.
__device__ __forceinline__ int hmir(int v) { return __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false); }
__device__ __forceinline__ int rmir(int v) { return __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false); }

// Cross-lane reductions on the VALU (DPP and readlane; ds_bpermute-based
// shuffles go through the LDS pipe, which the weight DMA keeps busy).  The
// max works on the bits of non-negative floats (same order, no NaN handling
// needed); integer sums are exact.  Every lane of the group gets the result;
// all 64 lanes must be active.
__device__ __forceinline__ uint32_t umax8(uint32_t v) {
    v = max(v, (uint32_t)qx1((int)v));
    v = max(v, (uint32_t)qx2((int)v));
    return max(v, (uint32_t)hmir((int)v));
}
__device__ __forceinline__ uint32_t umax64(uint32_t v) {
    v = umax8(v);
    v = max(v, (uint32_t)rmir((int)v));
    const uint32_t a = max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
    const uint32_t b = max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
    return max(a, b);
}
__device__ __forceinline__ int sum4i(int v) {
    v += qx1(v);
    return v + qx2(v);
}
__device__ __forceinline__ int sum8i(int v) {
    v = sum4i(v);
    return v + hmir(v);
}

// Plain 4-byte-aligned global loads (dword alignment is all gfx950 needs
// for multi-dword global loads).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ u32x4 ld4(const uint8_t * p) { return *(const u32x4 *)p; }
__device__ __forceinline__ uint32_t ld1(const uint8_t * p) { return *(const uint32_t *)p; }
__device__ __forceinline__ uint32_t ldh(const uint8_t * p) { return *(const uint16_t *)p; }
// streamed-once weight loads: non-temporal hint keeps them from evicting the
// reused activations from L2.
#ifndef FLH_NT
#define FLH_NT 1
#endif
__device__ __forceinline__ u32x4 ld4_nt(const uint8_t * p) {
#if FLH_NT
    return __builtin_nontemporal_load((const u32x4 *)p);
#else
    return *(const u32x4 *)p;
#endif
}

// bit i of the 4-bit n -> bit 0 of byte i
__device__ __forceinline__ uint32_t spread4(uint32_t n) { return (n * 0x00204081u) & 0x01010101u; }

// ---- IQ2_XXS / IQ3_XXS (reference src/runtime/quants.h:27-38, 231-290) ----
// A 256-element superblock: f16 d, then per 32-element group ib a 32-bit
// scale/sign word w1 (top nibble: scale s; four 7-bit sign fields) and the
// grid indices of its 8-element runs (IQ2: 4 index bytes before w1, 8
// magnitudes per entry; IQ3: 8 index bytes in a leading 64-byte array, 4 per
// entry, w1 words after it).  Group scale db = (d * (0.5 + s)) * 0.25 (IQ2)
// or * 0.5 (IQ3).  The 7-bit sign field of run l widens to a byte with an
// even-parity top bit; bit j negates element 8l + j.
static __device__ const uint64_t k_iq2_grid[256] = { FLH_IQ2XXS_GRID_VALUES };
static __device__ const uint32_t k_iq3_grid[256] = { FLH_IQ3XXS_GRID_VALUES };

__host__ __device__ constexpr uint32_t iq_block_bytes(int fmt) { return fmt == FMT_IQ2_XXS ? 66u : 98u; }
__device__ __forceinline__ uint32_t iq_sign8(uint32_t s7) {
    s7 &= 127u;
    return s7 | (((uint32_t)__builtin_popcount(s7) & 1u) << 7);
}
// bytewise negate of the bytes of v whose mask byte is 0xFF; v's bytes are
// grid magnitudes in [1, 127], so no byte borrows from its neighbour
__device__ __forceinline__ uint32_t iq_apply(uint32_t v, uint32_t neg) {
    return (v ^ neg) + (neg & 0x01010101u);
}
__device__ __forceinline__ uint32_t iq_neg4(uint32_t bits4) { return spread4(bits4 & 0xFu) * 0xFFu; }
__device__ __forceinline__ uint32_t iq_ldu32(const uint8_t * p) {
    return p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24);
}
// scale/sign word of group ib of superblock b
__device__ __forceinline__ uint32_t iq_w1(int fmt, const uint8_t * b, int ib) {
    return fmt == FMT_IQ2_XXS ? iq_ldu32(b + 2 + 8 * ib + 4) : iq_ldu32(b + 66 + 4 * ib);
}
__device__ __forceinline__ float iq_db(int fmt, float d, uint32_t w1) {
    return fmt == FMT_IQ2_XXS ? d * (0.5f + (float)(w1 >> 28)) * 0.25f
                              : d * (0.5f + (float)(w1 >> 28)) * 0.5f;
}
// signed magnitude of element e (0..31) of group ib
__device__ __forceinline__ int iq_val(int fmt, const uint8_t * b, int ib, uint32_t w1, int e) {
    const int l = e >> 3, j = e & 7;
    const uint32_t s = iq_sign8(w1 >> (7 * l));
    int v;
    if (fmt == FMT_IQ2_XXS) {
        const uint32_t w0 = iq_ldu32(b + 2 + 8 * ib);
        v = (int)((k_iq2_grid[(w0 >> (8 * l)) & 0xFFu] >> (8 * j)) & 0xFFu);
    } else {
        v = (int)((k_iq3_grid[b[2 + 8 * ib + 2 * l + (j >> 2)]] >> (8 * (j & 3))) & 0xFFu);
    }
    return (s >> j) & 1u ? -v : v;
}

// ROUTER_SEL of one token by one wave (n_expert <= 64, top_k <= 8): lane i
// owns logit i; the same float operations in the same order as
// fl_op_router_sel (src/runtime/decode_params.h:234-265): max in ascending
// expert order (first strictly greater wins); expf; sum in ascending order;
// divide; top-k by first maximum; optional renormalisation by the sum of the
// chosen weights; scale.  Lane 0 writes ids[0..top_k) and, when gates is not
// null, gates[0..top_k) (generic pointers: global or LDS).  Every broadcast
// reads one uniformly indexed lane: v_readlane (scalar), not an LDS permute.
__device__ __forceinline__ void router_token_wave(const float * lg, uint32_t n_expert, uint32_t top_k,
                                                  uint32_t norm, float scale, uint32_t lane, uint32_t * ids,
                                                  float * gates) {
    const float l = lane < n_expert ? lg[lane] : 0.f;
    float mx = -1e30f;
    for (uint32_t i = 0; i < n_expert; ++i) {
        const float li = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), (int)i));
        if (li > mx) mx = li;
    }
    float w = lane < n_expert ? expf(l - mx) : 0.f;
    float sum = 0.f;
    for (uint32_t i = 0; i < n_expert; ++i) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), (int)i));
    w /= sum;
    bool taken = lane >= n_expert;
    float tsum = 0.f;
    uint32_t id_k[8];
    float gt_k[8];
    for (uint32_t k = 0; k < top_k; ++k) {
        // first lane holding the largest untaken weight (strict >, ascending)
        float bw = -1.f;
        uint32_t best = 0;
        for (uint32_t i = 0; i < n_expert; ++i) {
            const float wi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), (int)i));
            const bool ti = __builtin_amdgcn_readlane((int)taken, (int)i) != 0;
            if (!ti && wi > bw) { bw = wi; best = i; }
        }
        if (lane == best) taken = true;
        if (k < 8) { id_k[k] = best; gt_k[k] = bw; }
        tsum += bw;
    }
    if (lane == 0) {
        for (uint32_t k = 0; k < top_k && k < 8; ++k) {
            float g = gt_k[k];
            if (norm) g /= tsum;
            g *= scale;
            ids[k] = id_k[k];
            if (gates) gates[k] = g;
        }
    }
}

}  // namespace flh
