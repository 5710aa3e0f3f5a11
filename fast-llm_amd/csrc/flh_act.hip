// flh_act.hip -- ACT_Q8 (activation quantisation) and bit-exact dequant.
//
// ACT_Q8 writes, per column, the q8_1 appendix (per 32: f16 d, f16 s, i8 qs)
// and the q8_K appendix (per 256: f32 d, i16 bsums[16], i8 qs) with the same
// bytes as the reference's fl_quantize_q8_1_block / fl_quantize_q8_K_block
// (src/runtime/quants.h:360-416): amax is a max (order free), d = amax/127
// and id = 127/amax are correctly rounded IEEE divisions, q = roundf(x*id)
// clamped to +-127, sums are exact integers, halves are RNE.
//
// One wave per 256-element chunk of one column: lane i owns elements
// 4i..4i+3 (one 16-B load, one packed dword store per appendix); 8-lane
// groups form the q8_1 blocks, 4-lane groups the q8_K 16-sums.
#include "flh_kstream.h"
#include "flh_internal.h"
#include "flh_status.h"

namespace flh {

__global__ __launch_bounds__(64) void k_act_q8(float * x, uint8_t * yq, uint32_t cols,
                                               uint32_t xstride) {
    const uint32_t lane = threadIdx.x, chunk = blockIdx.x, col = blockIdx.y;
    float * xc = x + (size_t)col * xstride;
    uint8_t * q81 = yq ? yq + (size_t)col * xstride * 4 : (uint8_t *)xc + xq_off(cols);
    uint8_t * q8k = (uint8_t *)xc + xqk_off(cols);
    const uint32_t e0 = chunk * 256 + lane * 4;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (e0 + j < cols) ? xc[e0 + j] : 0.f;
    act_q8_lanes(v, lane, chunk, q81, q8k, cols);
}

// SILU_MUL fused with the ACT_Q8 of its output (the MoE / FFN down input):
// lane i of the wave for chunk `chunk` of column c computes h = silu(g) * u
// for elements 4i..4i+3 with k_silu_mul's expression, stores h, and quantises
// the same register values -- the bytes of k_silu_mul followed by k_act_q8.
__global__ __launch_bounds__(64) void k_silu_act_q8(const float * gate, const float * up, float * h, uint32_t n,
                                                    uint32_t gstride, uint32_t hstride) {
    const uint32_t lane = threadIdx.x, chunk = blockIdx.x, col = blockIdx.y;
    const float * gc = gate + (size_t)col * gstride;
    const float * uc = up + (size_t)col * gstride;
    float * hc = h + (size_t)col * hstride;
    const uint32_t e0 = chunk * 256 + lane * 4;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[j] = 0.f;
        if (e0 + j < n) {
            const float g = gc[e0 + j];
            v[j] = (g / (1.0f + expf(-g))) * uc[e0 + j];
            hc[e0 + j] = v[j];
        }
    }
    act_q8_lanes(v, lane, chunk, (uint8_t *)hc + xq_off(n), (uint8_t *)hc + xqk_off(n), n);
}

// RMSNORM of one column with (write_app) the ACT_Q8 of its output, one
// workgroup of 16 waves: the sum of squares as thread partials (elements
// 4t..4t+3, 4t+4096.. in order) -> a wave butterfly (xor_lane exchanges;
// every lane ends with the same sum) -> the 16 wave sums in wave order; s = 1 / sqrtf(ss / n + eps)
// (correctly rounded sqrt and division, as the reference's libm); then wave w
// quantises chunks w, w + 16, ... with y = (x * s) * wnorm computed in the
// registers it quantises, so the appendices hold ACT_Q8's bytes for the
// stored y.
__global__ __launch_bounds__(1024) void k_rmsnorm_act_q8(const float * x, const float * wn, float * y, uint32_t n,
                                                         float eps, int write_app) {
    __shared__ float part[16];
    __shared__ float sh_s;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float ss = 0.f;
    for (uint32_t e0 = 4 * tid; e0 < n; e0 += 4096)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (e0 + j < n) ss += x[e0 + j] * x[e0 + j];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) ss += xor_lane(ss, o, lane);
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    if (tid == 0) {
        float t = 0.f;
        for (int w = 0; w < 16; ++w) t += part[w];
        sh_s = 1.0f / sqrtf(t / (float)n + eps);
    }
    __syncthreads();
    const float s = sh_s;
    uint8_t * q81 = (uint8_t *)y + xq_off(n);
    uint8_t * q8k = (uint8_t *)y + xqk_off(n);
    for (uint32_t c = wave; c * 256 < n; c += 16) {
        const uint32_t e0 = c * 256 + 4 * lane;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j] = 0.f;
            if (e0 + j < n) {
                v[j] = x[e0 + j] * s * wn[e0 + j];
                y[e0 + j] = v[j];
            }
        }
        if (write_app) act_q8_lanes(v, lane, c, q81, q8k, n);
    }
}
// The same for n <= 16384, n % 4 == 0: thread t's elements (4t..4t+3,
// 4t+4096.., the chunks wave, wave + 16, ... of the loop above) and their
// norm weights come in as 16-B loads issued together, stay in registers
// through the reduction, and every thread sums the 16 wave partials itself
// (same order, so all hold the same s): one load round trip and one barrier.
__global__ __launch_bounds__(1024) void k_rmsnorm_act_q8_reg(const float * x, const float * wn, float * y, uint32_t n,
                                                             float eps, int write_app) {
    __shared__ float part[16];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float4 xv[4], wv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t e0 = 4 * tid + 4096 * k;
        if (e0 < n) {
            xv[k] = *(const float4 *)(x + e0);
            wv[k] = *(const float4 *)(wn + e0);
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (4 * tid + 4096 * k < n) {
            ss += xv[k].x * xv[k].x;
            ss += xv[k].y * xv[k].y;
            ss += xv[k].z * xv[k].z;
            ss += xv[k].w * xv[k].w;
        }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) ss += xor_lane(ss, o, lane);
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < 16; ++w) t += part[w];
    const float s = 1.0f / sqrtf(t / (float)n + eps);
    uint8_t * q81 = (uint8_t *)y + xq_off(n);
    uint8_t * q8k = (uint8_t *)y + xqk_off(n);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t c = wave + 16 * k, e0 = c * 256 + 4 * lane;
        if (c * 256 >= n) break;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (e0 < n) {
            v[0] = xv[k].x * s * wv[k].x;
            v[1] = xv[k].y * s * wv[k].y;
            v[2] = xv[k].z * s * wv[k].z;
            v[3] = xv[k].w * s * wv[k].w;
            *(float4 *)(y + e0) = make_float4(v[0], v[1], v[2], v[3]);
        }
        if (write_app) act_q8_lanes(v, lane, c, q81, q8k, n);
    }
}
int launch_rmsnorm_act_q8(const float * x, const float * wnorm, float * y, uint32_t n, float eps, bool app,
                          hipStream_t s) {
    if (n == 0) return FLH_OK;
    const bool reg = n <= 16384 && n % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)wnorm & 15) == 0 &&
                     ((uintptr_t)y & 15) == 0;
    if (reg)
        hipLaunchKernelGGL(k_rmsnorm_act_q8_reg, dim3(1), dim3(1024), 0, s, x, wnorm, y, n, eps, app ? 1 : 0);
    else
        hipLaunchKernelGGL(k_rmsnorm_act_q8, dim3(1), dim3(1024), 0, s, x, wnorm, y, n, eps, app ? 1 : 0);
    return hip_check(hipGetLastError(), "k_rmsnorm_act_q8 launch");
}
int launch_silu_act_q8(const float * gate, const float * up, float * h, uint32_t n, uint32_t ncol,
                       uint32_t gstride, uint32_t hstride, hipStream_t s) {
    if (n == 0 || ncol == 0) return FLH_OK;
    hipLaunchKernelGGL(k_silu_act_q8, dim3((n + 255) / 256, ncol), dim3(64), 0, s, gate, up, h, n, gstride, hstride);
    return hip_check(hipGetLastError(), "k_silu_act_q8 launch");
}

int launch_act_q8(float * x, void * y_q81, uint32_t cols, uint32_t nx,
                  uint32_t xstride, hipStream_t s) {
    if (cols == 0 || nx == 0) return FLH_OK;
    const uint32_t chunks = (cols + 255) / 256;
    hipLaunchKernelGGL(k_act_q8, dim3(chunks, nx), dim3(64), 0, s, x, (uint8_t *)y_q81,
                       cols, xstride);
    return hip_check(hipGetLastError(), "k_act_q8 launch");
}

// ---------------------------------------------------------------- dequant --
// Bit-exact restatement of dequant_chunk's value formulas; byte loads (this
// is a correctness/embedding path, not the streamed hot loop).  One thread
// per 32 outputs (Q8_0: a block; Q4_K: 16 nibble pairs; Q6_K: 16 positions x
// 4 groups... split as 32 outputs of one group pair).
__global__ void k_dequant(int fmt, const uint8_t * __restrict__ w, uint32_t rows,
                          uint32_t cols, float * __restrict__ out) {
    const uint64_t units_per_row = cols / 32;
    const uint64_t u = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units_per_row * rows) return;
    const uint32_t r = (uint32_t)(u / units_per_row), j = (uint32_t)(u % units_per_row);
    float * o = out + (size_t)r * cols;
    if (fmt == FMT_Q8_0) {
        const uint8_t * b = w + (size_t)r * (cols / 32) * 34 + (size_t)j * 34;
        const float d = h2f(b[0] | (b[1] << 8));
        for (int i = 0; i < 32; ++i) o[32 * j + i] = d * (float)(int8_t)b[2 + i];
    } else if (fmt == FMT_Q5_0) {
        const uint8_t * b = w + (size_t)r * (cols / 32) * 22 + (size_t)j * 22;
        const float d = h2f(b[0] | (b[1] << 8));
        const uint32_t qh = b[2] | (b[3] << 8) | (b[4] << 16) | ((uint32_t)b[5] << 24);
        for (int i = 0; i < 16; ++i) {
            const uint32_t lo = (b[6 + i] & 0x0F) | (((qh >> i) << 4) & 0x10);
            const uint32_t hi = (b[6 + i] >> 4) | ((qh >> (i + 12)) & 0x10);
            o[32 * j + i] = d * (float)((int)lo - 16);
            o[32 * j + 16 + i] = d * (float)((int)hi - 16);
        }
    } else if (fmt == FMT_Q4_K) {
        const uint32_t sb = j >> 3, g = j & 7, c = g >> 1;   // group g of superblock sb
        const uint8_t * b = w + (size_t)r * (cols / 256) * 144 + (size_t)sb * 144;
        const float d = h2f(b[0] | (b[1] << 8)), dmin = h2f(b[2] | (b[3] << 8));
        const uint8_t * s = b + 4;
        uint32_t sc, mn;
        if (g < 4) { sc = s[g] & 63; mn = s[g + 4] & 63; }
        else { sc = (s[g + 4] & 0xF) | ((s[g - 4] >> 6) << 4); mn = (s[g + 4] >> 4) | ((s[g] >> 6) << 4); }
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        const uint8_t * q = b + 16 + 32 * c;
        float * oo = o + 256 * sb + 64 * c + 32 * (g & 1);
        for (int l = 0; l < 32; ++l) {
            const uint32_t nib = (g & 1) ? (q[l] >> 4) : (q[l] & 0xF);
            oo[l] = d1 * (float)nib - m1;
        }
    } else if (fmt == FMT_IQ2_XXS || fmt == FMT_IQ3_XXS) {
        // group ib of superblock sb: db * (+-grid magnitude), the factor the
        // reference's canonical IQ dots multiply x by (quants.h:252-254,
        // 280-283); its dequant_chunk has no IQ case (kernels.h:215-221)
        const uint32_t sb = j >> 3, ib = j & 7, bb = iq_block_bytes(fmt);
        const uint8_t * b = w + (size_t)r * (cols / 256) * bb + (size_t)sb * bb;
        const uint32_t w1 = iq_w1(fmt, b, ib);
        const float db = iq_db(fmt, h2f(b[0] | (b[1] << 8)), w1);
        for (int e = 0; e < 32; ++e) o[32 * j + e] = db * (float)iq_val(fmt, b, ib, w1, e);
    } else {  // Q6_K: group (h, gg) of superblock sb, positions l < 32
        const uint32_t sb = j >> 3, h = (j >> 2) & 1, gg = j & 3;
        const uint8_t * b = w + (size_t)r * (cols / 256) * 210 + (size_t)sb * 210;
        const float d = h2f(b[208] | (b[209] << 8));
        const uint8_t * ql = b + 64 * h, * qh = b + 128 + 32 * h;
        const int8_t * sc = (const int8_t *)(b + 192) + 8 * h;
        float * oo = o + 256 * sb + 128 * h + 32 * gg;
        for (int l = 0; l < 32; ++l) {
            const uint8_t lb = ql[l + 32 * (gg & 1)];
            const int q6 = ((gg < 2) ? (lb & 0xF) : (lb >> 4)) | (((qh[l] >> (2 * gg)) & 3) << 4);
            oo[l] = d * (float)sc[l / 16 + 2 * gg] * (float)(q6 - 32);
        }
    }
}

int launch_dequant(int fmt, const uint8_t * w, uint32_t rows, uint32_t cols,
                   float * out, hipStream_t s) {
    if (fmt < FMT_Q8_0 || fmt > FMT_IQ3_XXS)
        return set_error(FLH_ERR_UNSUPPORTED, "dequant: format not supported");
    const uint64_t units = (uint64_t)rows * (cols / 32);
    if (units == 0) return FLH_OK;
    hipLaunchKernelGGL(k_dequant, dim3((uint32_t)((units + 255) / 256)), dim3(256), 0, s,
                       fmt, w, rows, cols, out);
    return hip_check(hipGetLastError(), "k_dequant launch");
}

}  // namespace flh
