// flh_quant.hip -- synthetic-weight generation: a counter-based normal
// generator and fp32 -> Q8_0 / Q4_K / Q6_K weight quantizers.
//
// The reference ships no weight quantizer (its weights come from GGUF
// files), so these are this backend's own.  They are simple single-pass
// min/max quantizers (not llama.cpp's iterative search): the kernels and the
// parity tests only need valid blocks with realistic statistics.  The block
// code is __host__ __device__ with identical float operations, so
// flh_quantize (device) and flh_quantize_host produce the same bytes.
#include "flh_common.h"
#include "flh_internal.h"
#include "flh_status.h"
#include <math.h>
#include <string.h>

namespace flh {

#define HD __host__ __device__

HD inline float qh2f(uint32_t h) {          // exact binary16 -> binary32
    const uint32_t sign = (h >> 15) << 31, exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu, bits;
    if (exp == 0x1Fu) bits = sign | 0x7F800000u | (man << 13);
    else if (exp) bits = sign | ((exp + 112u) << 23) | (man << 13);
    else if (!man) bits = sign;
    else {
        int e = 113;
        while (!(man & 0x400u)) { man <<= 1; --e; }
        bits = sign | ((uint32_t)e << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
HD inline uint32_t qf2h(float f) {          // RNE binary32 -> binary16
    uint32_t u;
    memcpy(&u, &f, 4);
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
HD inline float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
HD inline void st16(uint8_t * p, uint32_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

HD void quant_q8_0_block(const float * x, uint8_t * o) {
    float amax = 0.f;
    for (int i = 0; i < 32; ++i) amax = fabsf(x[i]) > amax ? fabsf(x[i]) : amax;
    const float d = amax / 127.f, id = amax > 0.f ? 127.f / amax : 0.f;
    st16(o, qf2h(d));
    for (int i = 0; i < 32; ++i) o[2 + i] = (uint8_t)(int8_t)clampf(roundf(x[i] * id), -127.f, 127.f);
}

HD void quant_q4_K_block(const float * x, uint8_t * o) {
    float scl[8], mnv[8], maxs = 0.f, maxm = 0.f;
    for (int j = 0; j < 8; ++j) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int l = 1; l < 32; ++l) {
            const float v = x[32 * j + l];
            lo = v < lo ? v : lo;
            hi = v > hi ? v : hi;
        }
        if (lo > 0.f) lo = 0.f;
        scl[j] = (hi - lo) / 15.f;
        mnv[j] = -lo;
        maxs = scl[j] > maxs ? scl[j] : maxs;
        maxm = mnv[j] > maxm ? mnv[j] : maxm;
    }
    const uint32_t dh = qf2h(maxs / 63.f), mh = qf2h(maxm / 63.f);
    const float d = qh2f(dh), dmin = qh2f(mh);
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = d > 0.f ? (uint8_t)clampf(roundf(scl[j] / d), 0.f, 63.f) : 0;
        mn[j] = dmin > 0.f ? (uint8_t)clampf(roundf(mnv[j] / dmin), 0.f, 63.f) : 0;
    }
    st16(o, dh);
    st16(o + 2, mh);
    uint8_t * s = o + 4;   // inverse of the 6-bit unpack (quants.h:121-129)
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; ++j) {
        const float ds = d * (float)sc[j], dm = dmin * (float)mn[j];
        for (int l = 0; l < 32; ++l)
            q[32 * j + l] = ds > 0.f ? (uint8_t)clampf(roundf((x[32 * j + l] + dm) / ds), 0.f, 15.f) : 0;
    }
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l)
            o[16 + 32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

HD void quant_q6_K_block(const float * x, uint8_t * o) {
    float scl[16], maxs = 0.f;
    for (int i = 0; i < 16; ++i) {
        float a = 0.f;
        for (int l = 0; l < 16; ++l) a = fabsf(x[16 * i + l]) > a ? fabsf(x[16 * i + l]) : a;
        scl[i] = a / 31.f;
        maxs = scl[i] > maxs ? scl[i] : maxs;
    }
    const uint32_t dh = qf2h(maxs / 127.f);
    const float d = qh2f(dh);
    int8_t sc[16];
    for (int i = 0; i < 16; ++i)
        sc[i] = d > 0.f ? (int8_t)clampf(roundf(scl[i] / d), -127.f, 127.f) : 0;
    memset(o, 0, 210);
    for (int e = 0; e < 256; ++e) {
        const float ds = d * (float)sc[e / 16];
        const int q = ds > 0.f ? (int)clampf(roundf(x[e] / ds), -32.f, 31.f) : 0;
        const uint32_t q6 = (uint32_t)(q + 32);
        const int h = e / 128, g = (e % 128) / 32, l = e % 32;
        uint8_t & lb = o[64 * h + l + 32 * (g & 1)];
        lb |= (uint8_t)(g < 2 ? (q6 & 0xF) : ((q6 & 0xF) << 4));
        o[128 + 32 * h + l] |= (uint8_t)((q6 >> 4) << (2 * g));
    }
    for (int i = 0; i < 16; ++i) o[192 + i] = (uint8_t)sc[i];
    st16(o + 208, dh);
}

HD inline void quant_block(int fmt, const float * x, uint8_t * o) {
    if (fmt == FMT_Q8_0) quant_q8_0_block(x, o);
    else if (fmt == FMT_Q4_K) quant_q4_K_block(x, o);
    else quant_q6_K_block(x, o);
}
inline uint32_t blk_elems(int fmt) { return fmt == FMT_Q8_0 ? 32u : 256u; }
inline uint32_t blk_bytes(int fmt) { return fmt == FMT_Q8_0 ? 34u : fmt == FMT_Q4_K ? 144u : 210u; }

__global__ void k_quantize(int fmt, const float * src, uint64_t nblk, uint32_t be,
                           uint32_t bb, uint8_t * dst) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    quant_block(fmt, src + i * be, dst + i * bb);
}

static int check_fmt(int fmt, uint32_t cols) {
    if (fmt != FMT_Q8_0 && fmt != FMT_Q4_K && fmt != FMT_Q6_K)
        return set_error(FLH_ERR_UNSUPPORTED, "quantize: format not supported");
    if (cols % blk_elems(fmt)) return set_error(FLH_ERR_ARG, "quantize: cols not a multiple of the block");
    return FLH_OK;
}

int launch_quantize_weights(int fmt, const float * src, uint32_t rows, uint32_t cols,
                            uint8_t * dst, hipStream_t s) {
    if (int rc = check_fmt(fmt, cols)) return rc;
    const uint64_t nblk = (uint64_t)rows * (cols / blk_elems(fmt));
    if (nblk == 0) return FLH_OK;
    hipLaunchKernelGGL(k_quantize, dim3((uint32_t)((nblk + 127) / 128)), dim3(128), 0, s, fmt,
                       src, nblk, blk_elems(fmt), blk_bytes(fmt), dst);
    return hip_check(hipGetLastError(), "k_quantize launch");
}

int quantize_host(int fmt, const float * src, uint32_t rows, uint32_t cols, uint8_t * dst) {
    if (int rc = check_fmt(fmt, cols)) return rc;
    const uint64_t nblk = (uint64_t)rows * (cols / blk_elems(fmt));
    for (uint64_t i = 0; i < nblk; ++i)
        quant_block(fmt, src + i * blk_elems(fmt), dst + i * blk_bytes(fmt));
    return FLH_OK;
}

// ------------------------------------------------------- normal generator --
__device__ inline uint64_t mix64(uint64_t z) {      // splitmix64 finaliser
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void k_fill_normal(float * dst, uint64_t n, uint64_t seed, float mean, float sd,
                              uint32_t out_thr, float out_scale) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t h = mix64(seed * 0x100000001B3ull ^ mix64(i));
    const float u1 = ((float)((h >> 40) & 0xFFFFFF) + 0.5f) * (1.0f / 16777216.0f);
    const float u2 = (float)((h >> 16) & 0xFFFFFF) * (1.0f / 16777216.0f);
    float z = sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2);
    if ((uint32_t)(h & 0xFFFF) < out_thr) z *= out_scale;
    dst[i] = mean + sd * z;
}

int launch_fill_normal(float * dst, size_t n, uint64_t seed, float mean, float stddev,
                       float outlier_frac, float outlier_scale, hipStream_t s) {
    if (n == 0) return FLH_OK;
    const uint32_t thr = (uint32_t)(clampf(outlier_frac, 0.f, 1.f) * 65536.f);
    hipLaunchKernelGGL(k_fill_normal, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, dst,
                       (uint64_t)n, seed, mean, stddev, thr, outlier_scale);
    return hip_check(hipGetLastError(), "k_fill_normal launch");
}

}  // namespace flh
