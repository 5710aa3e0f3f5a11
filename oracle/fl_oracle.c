/*
 * fl_oracle.c -- CPU restatement of the reference quantized-dot path.
 * TEST INFRASTRUCTURE ONLY (see fl_oracle.h): the checker, never the product.
 *
 * Build: cc -O2 -ffp-contract=off -fPIC -shared (oracle/Makefile).  The
 * arithmetic order of every float expression below is the order of the cited
 * reference line; -ffp-contract=off keeps a*b+c as two roundings, and every
 * fused step is an explicit fmaf, as in the reference.
 *
 * Block byte layouts (src/runtime/quants.h:23-26), read by offset here:
 *   Q8_0 34 B : d f16 @0, qs[32] i8 @2
 *   Q4_K 144 B: d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16
 *   Q6_K 210 B: ql[128] @0, qh[64] @128, scales[16] i8 @192, d f16 @208
 *   q8_1 36 B : d f16 @0, s f16 @2, qs[32] @4          (quants.h:299)
 *   q8_K 292 B: d f32 @0, bsums[16] i16 @4, qs[256] @36 (quants.h:316)
 */
#include "fl_oracle.h"
#include "../fast-llm_amd/csrc/flh_iq_grids.h"
#include <math.h>
#include <string.h>
#include <stdlib.h>
#include <pthread.h>

static uint16_t rd16(const uint8_t * p) { uint16_t v; memcpy(&v, p, 2); return v; }
static int16_t  rdi16(const uint8_t * p) { int16_t v; memcpy(&v, p, 2); return v; }
static float    rdf32(const uint8_t * p) { float v; memcpy(&v, p, 4); return v; }

/* IEEE binary16 -> binary32, exact (src/runtime/quants.h:40-64). */
float orc_half2float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {
        /* subnormal: value = man * 2^-24; normalise the mantissa */
        int e = 113;                    /* biased exponent of 2^-14 */
        while (!(man & 0x400u)) { man <<= 1; --e; }
        bits = sign | ((uint32_t)e << 23) | ((man & 0x3FFu) << 13);
    }
    float f; memcpy(&f, &bits, 4); return f;
}

/* binary32 -> binary16, round to nearest even (src/runtime/quants.h:333-356);
 * NaN -> 0x7E00|sign, overflow -> inf. */
uint16_t orc_float2half(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a >= 0x47800000u)                         /* >= 65536, inf, nan */
        return (uint16_t)(sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (a < 0x38800000u) {                        /* below 2^-14: subnormal */
        uint32_t e = a >> 23;
        if (e < 102) return (uint16_t)sign;       /* < 2^-25: rounds to 0 */
        uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
        uint32_t sh = 126u - e;                   /* 14..24 */
        uint32_t q = m >> sh, r = m & ((1u << sh) - 1u), hb = 1u << (sh - 1);
        if (r > hb || (r == hb && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((a >> 23) - 112u) << 10 | ((a >> 13) & 0x3FFu);
    uint32_t r = a & 0x1FFFu;
    if (r > 0x1000u || (r == 0x1000u && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

/* src/runtime/quants.h:76-99 */
uint32_t orc_blk_elems(int fmt) {
    switch (fmt) { case ORC_Q8_0: case ORC_Q5_0: return 32;
                   case ORC_Q4_K: case ORC_Q6_K: case ORC_IQ2_XXS: case ORC_IQ3_XXS: return 256;
                   default: return 1; }
}
uint32_t orc_blk_bytes(int fmt) {
    switch (fmt) { case ORC_Q8_0: return 34; case ORC_Q5_0: return 22;
                   case ORC_Q4_K: return 144; case ORC_Q6_K: return 210;
                   case ORC_IQ2_XXS: return 66; case ORC_IQ3_XXS: return 98;
                   default: return 4; }
}

/* ---- IQ2_XXS / IQ3_XXS codebook formats (src/runtime/quants.h:27-38,
 *      231-290).  Per 32-element group ib of a 256-element superblock: a
 *      4-bit scale s (top nibble of the group's 32-bit sign/scale word w1)
 *      gives db = (d * (0.5 + s)) * 0.25 (IQ2) or * 0.5 (IQ3); four 7-bit
 *      sign fields of w1 widen to sign bytes with an even-parity top bit
 *      (the format's sign table). */
static const uint64_t iq2_grid[256] = { FLH_IQ2XXS_GRID_VALUES };
static const uint32_t iq3_grid[256] = { FLH_IQ3XXS_GRID_VALUES };
uint8_t orc_iq_signs(uint32_t s7) {
    s7 &= 127u;
    return (uint8_t)(s7 | ((uint32_t)__builtin_parity(s7) << 7));
}
uint64_t orc_iq2_grid(int i) { return iq2_grid[i & 255]; }
uint32_t orc_iq3_grid(int i) { return iq3_grid[i & 255]; }
static uint32_t rd32(const uint8_t * p) { uint32_t v; memcpy(&v, p, 4); return v; }
/* group ib's scale-sign word and its grid magnitude of element e (0..31) */
static uint32_t iq_w1(int fmt, const uint8_t * b, int ib) {
    return fmt == ORC_IQ2_XXS ? rd32(b + 2 + 8 * ib + 4) : rd32(b + 2 + 64 + 4 * ib);
}
static float iq_db(int fmt, const uint8_t * b, uint32_t w1) {
    const float d = orc_half2float(rd16(b));
    return fmt == ORC_IQ2_XXS ? d * (0.5f + (float)(w1 >> 28)) * 0.25f
                              : d * (0.5f + (float)(w1 >> 28)) * 0.5f;
}
/* signed magnitude of element e of group ib (grid byte, sign from the
 * group's l-th sign byte; IQ3 entries 2l / 2l+1 take sign bits 0-3 / 4-7) */
static int iq_val(int fmt, const uint8_t * b, int ib, int e) {
    const uint32_t w1 = iq_w1(fmt, b, ib);
    const int l = e >> 3, j = e & 7;
    const uint8_t s = orc_iq_signs(w1 >> (7 * l));
    int v;
    if (fmt == ORC_IQ2_XXS) {
        const uint32_t w0 = rd32(b + 2 + 8 * ib);
        v = (int)(uint8_t)(iq2_grid[(w0 >> (8 * l)) & 0xFF] >> (8 * j));
    } else {
        const uint8_t * qs = b + 2;
        v = (int)(uint8_t)(iq3_grid[qs[8 * ib + 2 * l + (j >> 2)]] >> (8 * (j & 3)));
    }
    return (s >> j) & 1 ? -v : v;
}
uint64_t orc_row_bytes(int fmt, uint32_t cols) {
    return (uint64_t)(cols / orc_blk_elems(fmt)) * orc_blk_bytes(fmt);
}

/* 6-bit scale/min unpack of Q4_K sub-block j (src/runtime/quants.h:121-129) */
void orc_q4k_scale_min(int j, const uint8_t * s, uint8_t * d, uint8_t * m) {
    if (j < 4) {
        *d = s[j] & 63u;
        *m = s[j + 4] & 63u;
    } else {
        *d = (uint8_t)((s[j + 4] & 0x0Fu) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* appendix offsets (src/runtime/quants.h:302-330) */
size_t orc_xq_offset(uint32_t cols) { return ((size_t)cols * 4 + 15) & ~(size_t)15; }
size_t orc_xqk_offset(uint32_t cols) {
    return orc_xq_offset(cols) + ((((size_t)cols / 32) * 36 + 15) & ~(size_t)15);
}
size_t orc_x_alloc_bytes(uint32_t cols) {
    return orc_xqk_offset(cols) + ((size_t)cols / 256) * 292;
}

/* ---- dequant (src/runtime/kernels.h:162-242) -------------------------- */
static void dq_q8_0(const uint8_t * b, float * o) {
    const float d = orc_half2float(rd16(b));
    for (int j = 0; j < 32; ++j) o[j] = d * (float)(int8_t)b[2 + j];
}
static void dq_q4_K(const uint8_t * b, float * o) {
    const float d = orc_half2float(rd16(b)), dmin = orc_half2float(rd16(b + 2));
    const uint8_t * sc = b + 4, * q = b + 16;
    for (int c = 0; c < 4; ++c) {                 /* 64-element chunks */
        uint8_t s0, m0, s1, m1;
        orc_q4k_scale_min(2 * c, sc, &s0, &m0);
        orc_q4k_scale_min(2 * c + 1, sc, &s1, &m1);
        const float d1 = d * (float)s0, mm1 = dmin * (float)m0;
        const float d2 = d * (float)s1, mm2 = dmin * (float)m1;
        for (int l = 0; l < 32; ++l) o[64 * c + l]      = d1 * (float)(q[32 * c + l] & 0xF) - mm1;
        for (int l = 0; l < 32; ++l) o[64 * c + 32 + l] = d2 * (float)(q[32 * c + l] >> 4) - mm2;
    }
}
/* Q5_0 element j of a block: 4 bits from qs, the 5th from qh (bit j) minus 16
 * (src/runtime/kernels.h:169-180, quants.h:144-162) */
static int q5_val(const uint8_t * b, int j) {
    const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
    const uint8_t * qs = b + 6;
    if (j < 16) return (int)((qs[j] & 0x0F) | (((qh >> j) << 4) & 0x10)) - 16;
    return (int)((qs[j - 16] >> 4) | ((qh >> (j - 16 + 12)) & 0x10)) - 16;
}
static void dq_q5_0(const uint8_t * b, float * o) {
    const float d = orc_half2float(rd16(b));
    for (int j = 0; j < 32; ++j) o[j] = d * (float)q5_val(b, j);
}
/* the 6-bit value of Q6_K element (half h, group g in 0..3, position l) */
static int q6_val(const uint8_t * b, int h, int g, int l) {
    const uint8_t * ql = b + 64 * h, * qh = b + 128 + 32 * h;
    const uint8_t lb = ql[l + 32 * (g & 1)];
    const int lo = (g < 2) ? (lb & 0xF) : (lb >> 4);
    return lo | (((qh[l] >> (2 * g)) & 3) << 4);
}
/* IQ dequant: element value db * (+-v), the factor fl_dot_row_iq2_xxs /
 * fl_dot_row_iq3_xxs multiply x by (src/runtime/quants.h:252-254, 280-283).
 * The reference's dequant_chunk has no IQ case (it zero-fills,
 * src/runtime/kernels.h:215-221); this defines the fp32 values. */
static void dq_iq(int fmt, const uint8_t * b, float * o) {
    for (int ib = 0; ib < 8; ++ib) {
        const float db = iq_db(fmt, b, iq_w1(fmt, b, ib));
        for (int e = 0; e < 32; ++e) {
            const int v = iq_val(fmt, b, ib, e);
            o[32 * ib + e] = db * (float)v;
        }
    }
}
static void dq_q6_K(const uint8_t * b, float * o) {
    const float d = orc_half2float(rd16(b + 208));
    const int8_t * sc = (const int8_t *)(b + 192);
    for (int h = 0; h < 2; ++h)
        for (int g = 0; g < 4; ++g)
            for (int l = 0; l < 32; ++l)
                o[128 * h + 32 * g + l] = d * (float)sc[8 * h + 2 * g + l / 16]
                                        * (float)(q6_val(b, h, g, l) - 32);
}

void orc_dequant_chunk(int fmt, const uint8_t * row, uint32_t elem0,
                       uint32_t n, float * out) {
    const uint32_t be = orc_blk_elems(fmt), bb = orc_blk_bytes(fmt);
    const uint8_t * bp = row + (size_t)(elem0 / be) * bb;
    if (fmt == ORC_F32) { memcpy(out, (const float *)row + elem0, (size_t)n * 4); return; }
    for (uint32_t b = 0; b < n / be; ++b) {
        const uint8_t * blk = bp + (size_t)b * bb;
        float * o = out + (size_t)b * be;
        if (fmt == ORC_Q8_0) dq_q8_0(blk, o);
        else if (fmt == ORC_Q5_0) dq_q5_0(blk, o);
        else if (fmt == ORC_Q4_K) dq_q4_K(blk, o);
        else if (fmt == ORC_Q6_K) dq_q6_K(blk, o);
        else if (fmt == ORC_IQ2_XXS || fmt == ORC_IQ3_XXS) dq_iq(fmt, blk, o);
    }
}
void orc_dequant_rows(int fmt, const uint8_t * w, uint32_t rows,
                      uint32_t cols, float * out) {
    const uint64_t rb = orc_row_bytes(fmt, cols);
    for (uint32_t r = 0; r < rows; ++r)
        orc_dequant_chunk(fmt, w + r * rb, 0, cols, out + (size_t)r * cols);
}

/* ---- canonical fp32-x dots, one accumulator, ascending elements
 *      (src/runtime/quants.h:132-230, 625-642) ------------------------------ */
static float dot_row_q8_0(const uint8_t * row, const float * x, uint32_t cols) {
    float acc = 0.f;
    for (uint32_t b = 0; b < cols / 32; ++b) {
        const uint8_t * B = row + (size_t)b * 34;
        const float d = orc_half2float(rd16(B));
        for (int i = 0; i < 32; ++i) acc += d * (float)(int8_t)B[2 + i] * x[b * 32 + i];
    }
    return acc;
}
/* src/runtime/quants.h:144-162: elements 0..15 (low nibbles) then 16..31 */
static float dot_row_q5_0(const uint8_t * row, const float * x, uint32_t cols) {
    float acc = 0.f;
    for (uint32_t b = 0; b < cols / 32; ++b) {
        const uint8_t * B = row + (size_t)b * 22;
        const float d = orc_half2float(rd16(B));
        for (int j = 0; j < 32; ++j) acc += d * (float)q5_val(B, j) * x[b * 32 + j];
    }
    return acc;
}
static float dot_row_q4_K(const uint8_t * row, const float * x, uint32_t cols) {
    float acc = 0.f;
    for (uint32_t sb = 0; sb < cols / 256; ++sb) {
        const uint8_t * B = row + (size_t)sb * 144;
        const float d = orc_half2float(rd16(B)), dmin = orc_half2float(rd16(B + 2));
        const uint8_t * q = B + 16;
        for (int c = 0; c < 4; ++c) {
            uint8_t s0, m0, s1, m1;
            orc_q4k_scale_min(2 * c, B + 4, &s0, &m0);
            orc_q4k_scale_min(2 * c + 1, B + 4, &s1, &m1);
            const float d1 = d * (float)s0, mm1 = dmin * (float)m0;
            const float d2 = d * (float)s1, mm2 = dmin * (float)m1;
            const float * xb = x + sb * 256 + 64 * c;
            for (int l = 0; l < 32; ++l) acc += (d1 * (float)(q[32 * c + l] & 0xF) - mm1) * xb[l];
            for (int l = 0; l < 32; ++l) acc += (d2 * (float)(q[32 * c + l] >> 4) - mm2) * xb[32 + l];
        }
    }
    return acc;
}
static float dot_row_q6_K(const uint8_t * row, const float * x, uint32_t cols) {
    float acc = 0.f;
    for (uint32_t sb = 0; sb < cols / 256; ++sb) {
        const uint8_t * B = row + (size_t)sb * 210;
        const float d = orc_half2float(rd16(B + 208));
        const int8_t * sc = (const int8_t *)(B + 192);
        for (int h = 0; h < 2; ++h)
            for (int g = 0; g < 4; ++g)
                for (int l = 0; l < 32; ++l)
                    acc += d * (float)sc[8 * h + 2 * g + l / 16]
                         * (float)(q6_val(B, h, g, l) - 32)
                         * x[sb * 256 + 128 * h + 32 * g + l];
    }
    return acc;
}
/* fl_dot_row_iq2_xxs / fl_dot_row_iq3_xxs (src/runtime/quants.h:237-290):
 * one accumulator; acc += (db * (+-v)) * x.  IQ2 walks elements ascending;
 * IQ3 interleaves the two grid entries of each 8-element run (element
 * 8l+j, then 8l+j+4, for j = 0..3). */
static float dot_row_iq(int fmt, const uint8_t * row, const float * x, uint32_t cols) {
    float acc = 0.f;
    const uint32_t bb = orc_blk_bytes(fmt);
    for (uint32_t sb = 0; sb < cols / 256; ++sb) {
        const uint8_t * B = row + (size_t)sb * bb;
        const float * xb = x + (size_t)sb * 256;
        for (int ib = 0; ib < 8; ++ib) {
            const float db = iq_db(fmt, B, iq_w1(fmt, B, ib));
            for (int l = 0; l < 4; ++l) {
                if (fmt == ORC_IQ2_XXS) {
                    for (int j = 0; j < 8; ++j) {
                        const int e = 8 * l + j;
                        acc += db * (float)iq_val(fmt, B, ib, e) * xb[32 * ib + e];
                    }
                } else {
                    for (int j = 0; j < 4; ++j) {
                        const int e1 = 8 * l + j, e2 = 8 * l + j + 4;
                        acc += db * (float)iq_val(fmt, B, ib, e1) * xb[32 * ib + e1];
                        acc += db * (float)iq_val(fmt, B, ib, e2) * xb[32 * ib + e2];
                    }
                }
            }
        }
    }
    return acc;
}

float orc_dot_row(int fmt, const uint8_t * row, const float * x, uint32_t cols) {
    switch (fmt) {
        case ORC_F32: {
            const float * r = (const float *)row; float acc = 0.f;
            for (uint32_t c = 0; c < cols; ++c) acc += r[c] * x[c];
            return acc;
        }
        case ORC_Q8_0: return dot_row_q8_0(row, x, cols);
        case ORC_Q5_0: return dot_row_q5_0(row, x, cols);
        case ORC_Q4_K: return dot_row_q4_K(row, x, cols);
        case ORC_Q6_K: return dot_row_q6_K(row, x, cols);
        case ORC_IQ2_XXS: case ORC_IQ3_XXS: return dot_row_iq(fmt, row, x, cols);
    }
    return 0.f;
}

/* ---- "fast" fp32 order: 16 lane partials, fixed tree
 *      (src/runtime/kernels.h:11-19, 59-104 scalar branch) ------------------ */
static float tree16(const float * L) {
    float s[4];
    for (int j = 0; j < 4; ++j) s[j] = (L[j] + L[4 + j]) + (L[8 + j] + L[12 + j]);
    return (s[0] + s[1]) + (s[2] + s[3]);
}
float orc_dot_row_fast(const float * row, const float * x, uint32_t cols) {
    const uint32_t n16 = cols & ~15u;
    float L[16] = {0};
    for (uint32_t k = 0; k < n16; k += 16)
        for (int j = 0; j < 16; ++j) L[j] += row[k + j] * x[k + j];
    const float head = tree16(L);
    float tail = 0.f;
    for (uint32_t k = n16; k < cols; ++k) tail += row[k] * x[k];
    return head + tail;
}
/* src/runtime/kernels.h:111-160 (scalar branch) */
float orc_dot_row_fast_q8_0(const uint8_t * row, const float * x, uint32_t cols) {
    float L[16] = {0};
    for (uint32_t b = 0; b < cols / 32; ++b) {
        const uint8_t * B = row + (size_t)b * 34;
        const float d = orc_half2float(rd16(B));
        for (int g = 0; g < 8; ++g)
            for (int j = 0; j < 4; ++j)
                L[(g & 3) * 4 + j] += d * (float)(int8_t)B[2 + g * 4 + j] * x[b * 32 + g * 4 + j];
    }
    return tree16(L);
}
/* src/runtime/kernels.h:244-254 */
float orc_dot_row_fast_dequant(int fmt, const uint8_t * row, const float * x,
                               uint32_t cols) {
    float buf[256], acc = 0.f;
    for (uint32_t e = 0; e < cols; e += 256) {
        const uint32_t n = (cols - e < 256) ? cols - e : 256;
        orc_dequant_chunk(fmt, row, e, n, buf);
        acc += orc_dot_row_fast(buf, x + e, n);
    }
    return acc;
}

/* ---- activation quantizers (src/runtime/quants.h:360-416) ------------- */
static float amax_of(const float * x, int n) {
    float a = 0.f;
    for (int i = 0; i < n; ++i) { const float v = fabsf(x[i]); if (v > a) a = v; }
    return a;
}
static int8_t q8_of(float v, float id) {
    float q = roundf(v * id);              /* round half away from zero */
    if (q > 127.f) q = 127.f;
    if (q < -127.f) q = -127.f;
    return (int8_t)q;
}
void orc_quantize_q8_1_block(const float * x, uint8_t * o) {
    const float amax = amax_of(x, 32);
    const float d = amax / 127.f;
    const float id = amax > 0.f ? 127.f / amax : 0.f;
    int sum = 0;
    for (int i = 0; i < 32; ++i) { const int8_t q = q8_of(x[i], id); o[4 + i] = (uint8_t)q; sum += q; }
    const uint16_t hd = orc_float2half(d), hs = orc_float2half(d * (float)sum);
    memcpy(o, &hd, 2); memcpy(o + 2, &hs, 2);
}
void orc_quantize_q8_K_block(const float * x, uint8_t * o) {
    const float amax = amax_of(x, 256);
    const float d = amax / 127.f;
    const float id = amax > 0.f ? 127.f / amax : 0.f;
    for (int g = 0; g < 16; ++g) {
        int bs = 0;
        for (int i = 0; i < 16; ++i) {
            const int8_t q = q8_of(x[16 * g + i], id);
            o[36 + 16 * g + i] = (uint8_t)q; bs += q;
        }
        const int16_t b16 = (int16_t)bs;
        memcpy(o + 4 + 2 * g, &b16, 2);
    }
    memcpy(o, &d, 4);
}
void orc_act_q8(float * x, uint32_t cols) {
    uint8_t * base = (uint8_t *)x;
    for (uint32_t b = 0; b < cols / 32; ++b)
        orc_quantize_q8_1_block(x + b * 32, base + orc_xq_offset(cols) + (size_t)b * 36);
    for (uint32_t sb = 0; sb < cols / 256; ++sb)
        orc_quantize_q8_K_block(x + sb * 256, base + orc_xqk_offset(cols) + (size_t)sb * 292);
}

/* ---- int8 dots: exact integer partials, explicit fmaf folds into
 *      acc[t & 3], final (a0+a1)+(a2+a3) (src/runtime/quants.h:418-594) ---- */
static float fold4(const float * a) { return (a[0] + a[1]) + (a[2] + a[3]); }

float orc_dot_i8_q8_0(const uint8_t * row, const uint8_t * xq, uint32_t cols) {
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t b = 0; b < cols / 32; ++b) {
        const uint8_t * W = row + (size_t)b * 34, * X = xq + (size_t)b * 36;
        int idot = 0;
        for (int i = 0; i < 32; ++i) idot += (int)(int8_t)W[2 + i] * (int)(int8_t)X[4 + i];
        a[b & 3] = fmaf(orc_half2float(rd16(W)) * orc_half2float(rd16(X)),
                        (float)idot, a[b & 3]);
    }
    return fold4(a);
}
/* src/runtime/quants.h:449-466: per block idot over the 5-bit values
 * (unshifted), isum over the activation; term (idot - 16 * isum) */
float orc_dot_i8_q5_0(const uint8_t * row, const uint8_t * xq, uint32_t cols) {
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t b = 0; b < cols / 32; ++b) {
        const uint8_t * W = row + (size_t)b * 22, * X = xq + (size_t)b * 36;
        int idot = 0, isum = 0;
        for (int i = 0; i < 32; ++i) {
            idot += (q5_val(W, i) + 16) * (int)(int8_t)X[4 + i];
            isum += (int)(int8_t)X[4 + i];
        }
        a[b & 3] = fmaf(orc_half2float(rd16(W)) * orc_half2float(rd16(X)),
                        (float)(idot - 16 * isum), a[b & 3]);
    }
    return fold4(a);
}
/* IQ2_XXS / IQ3_XXS x q8_1.  No reference CPU counterpart: the reference
 * keeps codebook tiles off the CPU (fl_dot_i8_any returns 0 for them,
 * src/runtime/quants.h:612-620) and runs them on its GPU int8 kernels
 * (gdot_i8_iq2_xxs / gdot_i8_iq3_xxs, src/runtime/kernels_gpu.h:759-852),
 * whose sums are q8_1 dot products scaled by db * dx per 32-element group.
 * This build fixes the order the Q8_0 int8 dot uses: per group b the exact
 * integer dot of the signed grid magnitudes with the q8_1 quants, folded
 * acc[b & 3] = fmaf(db * dx, idot, .), then (a0 + a1) + (a2 + a3). */
float orc_dot_i8_iq(int fmt, const uint8_t * row, const uint8_t * xq, uint32_t cols) {
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    const uint32_t bb = orc_blk_bytes(fmt);
    for (uint32_t b = 0; b < cols / 32; ++b) {
        const uint8_t * B = row + (size_t)(b / 8) * bb, * X = xq + (size_t)b * 36;
        const int ib = (int)(b & 7);
        int idot = 0;
        for (int e = 0; e < 32; ++e) idot += iq_val(fmt, B, ib, e) * (int)(int8_t)X[4 + e];
        const float db = iq_db(fmt, B, iq_w1(fmt, B, ib));
        a[b & 3] = fmaf(db * orc_half2float(rd16(X)), (float)idot, a[b & 3]);
    }
    return fold4(a);
}
float orc_dot_i8_q4_K(const uint8_t * row, const uint8_t * xq, uint32_t cols) {
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t sb = 0; sb < cols / 256; ++sb) {
        const uint8_t * W = row + (size_t)sb * 144;
        const float d = orc_half2float(rd16(W)), dmin = orc_half2float(rd16(W + 2));
        for (int g = 0; g < 8; ++g) {
            uint8_t sc, mn;
            orc_q4k_scale_min(g, W + 4, &sc, &mn);
            const uint8_t * q = W + 16 + (g / 2) * 32;
            const uint8_t * X = xq + (size_t)(sb * 8 + g) * 36;
            int idot = 0, isum = 0;
            for (int i = 0; i < 32; ++i) {
                const int w4 = (g & 1) ? (q[i] >> 4) : (q[i] & 0xF);
                idot += w4 * (int8_t)X[4 + i];
                isum += (int8_t)X[4 + i];
            }
            const float dx = orc_half2float(rd16(X));
            a[g & 3] = fmaf(d * (float)sc * dx, (float)idot, a[g & 3]);
            a[g & 3] = fmaf(-(dmin * (float)mn) * dx, (float)isum, a[g & 3]);
        }
    }
    return fold4(a);
}
float orc_dot_i8_q6_K(const uint8_t * row, const uint8_t * xq, uint32_t cols) {
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t sb = 0; sb < cols / 256; ++sb) {
        const uint8_t * W = row + (size_t)sb * 210;
        const float d = orc_half2float(rd16(W + 208));
        const int8_t * sc = (const int8_t *)(W + 192);
        for (int h = 0; h < 2; ++h)
            for (int g = 0; g < 4; ++g) {
                const uint8_t * X = xq + (size_t)(sb * 8 + h * 4 + g) * 36;
                const float dx = orc_half2float(rd16(X));
                for (int k = 0; k < 2; ++k) {
                    int idot = 0, isum = 0;
                    for (int i = 0; i < 16; ++i) {
                        const int e = 16 * k + i;
                        idot += q6_val(W, h, g, e) * (int8_t)X[4 + e];
                        isum += (int8_t)X[4 + e];
                    }
                    const int t = (int)sc[8 * h + 2 * g + k] * (idot - 32 * isum);
                    const int ti = 8 * h + 2 * g + k;
                    a[ti & 3] = fmaf(d * dx, (float)t, a[ti & 3]);
                }
            }
    }
    return fold4(a);
}
float orc_dot_i8k_q4_K(const uint8_t * row, const uint8_t * xk, uint32_t cols) {
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t sb = 0; sb < cols / 256; ++sb) {
        const uint8_t * W = row + (size_t)sb * 144, * X = xk + (size_t)sb * 292;
        const float d = orc_half2float(rd16(W)), dmin = orc_half2float(rd16(W + 2));
        const float dk = rdf32(X);
        int32_t iacc = 0, imins = 0;
        for (int g = 0; g < 8; ++g) {
            uint8_t sc, mn;
            orc_q4k_scale_min(g, W + 4, &sc, &mn);
            const uint8_t * q = W + 16 + (g / 2) * 32;
            int idot = 0;
            for (int i = 0; i < 32; ++i)
                idot += ((g & 1) ? (q[i] >> 4) : (q[i] & 0xF)) * (int8_t)X[36 + 32 * g + i];
            iacc += (int)sc * idot;
            imins += (int)mn * ((int)rdi16(X + 4 + 4 * g) + (int)rdi16(X + 6 + 4 * g));
        }
        a[sb & 3] = fmaf(d * dk, (float)iacc, a[sb & 3]);
        a[sb & 3] = fmaf(-(dmin * dk), (float)imins, a[sb & 3]);
    }
    return fold4(a);
}
float orc_dot_i8k_q6_K(const uint8_t * row, const uint8_t * xk, uint32_t cols) {
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t sb = 0; sb < cols / 256; ++sb) {
        const uint8_t * W = row + (size_t)sb * 210, * X = xk + (size_t)sb * 292;
        const float d = orc_half2float(rd16(W + 208)), dk = rdf32(X);
        const int8_t * sc = (const int8_t *)(W + 192);
        int32_t iacc = 0;
        for (int h = 0; h < 2; ++h)
            for (int g = 0; g < 4; ++g)
                for (int k = 0; k < 2; ++k) {
                    int idot = 0;
                    for (int i = 0; i < 16; ++i) {
                        const int e = 16 * k + i;
                        idot += q6_val(W, h, g, e) * (int8_t)X[36 + 32 * (4 * h + g) + e];
                    }
                    const int bs = rdi16(X + 4 + 2 * (2 * (4 * h + g) + k));
                    iacc += (int)sc[8 * h + 2 * g + k] * (idot - 32 * bs);
                }
        a[sb & 3] = fmaf(d * dk, (float)iacc, a[sb & 3]);
    }
    return fold4(a);
}

/* ---- exec_task_cpu STREAM_DOT routing (src/runtime/kernels.h:1037-1257;
 *      x86 has no NEON branch, shadow is off by default) -------------------- */
static float one_dot(int fmt, const uint8_t * row, const float * x, uint32_t cols,
                     int fast, uint32_t i8_mask, uint32_t i8k_mask) {
    if (!fast) return orc_dot_row(fmt, row, x, cols);
    if ((fmt == ORC_Q4_K || fmt == ORC_Q6_K) && ((i8k_mask >> fmt) & 1u)) {
        const uint8_t * xk = (const uint8_t *)x + orc_xqk_offset(cols);
        return fmt == ORC_Q4_K ? orc_dot_i8k_q4_K(row, xk, cols)
                               : orc_dot_i8k_q6_K(row, xk, cols);
    }
    if (fmt != ORC_F32 && ((i8_mask >> fmt) & 1u)) {
        const uint8_t * xq = (const uint8_t *)x + orc_xq_offset(cols);
        switch (fmt) {
            case ORC_Q8_0: return orc_dot_i8_q8_0(row, xq, cols);
            case ORC_Q5_0: return orc_dot_i8_q5_0(row, xq, cols);
            case ORC_Q4_K: return orc_dot_i8_q4_K(row, xq, cols);
            case ORC_Q6_K: return orc_dot_i8_q6_K(row, xq, cols);
            case ORC_IQ2_XXS: case ORC_IQ3_XXS: return orc_dot_i8_iq(fmt, row, xq, cols);
            default: return 0.f;
        }
    }
    switch (fmt) {
        case ORC_F32: return orc_dot_row_fast((const float *)row, x, cols);
        case ORC_Q8_0: return orc_dot_row_fast_q8_0(row, x, cols);
        default: return orc_dot_row_fast_dequant(fmt, row, x, cols);
    }
}

void orc_stream_dot(int fmt, const uint8_t * w, uint32_t rows, uint32_t cols,
                    const float * x, float * y, uint32_t nx, uint32_t xstride,
                    uint32_t ystride, int fast, uint32_t i8_mask,
                    uint32_t i8k_mask) {
    const uint64_t rb = fmt == ORC_F32 ? (uint64_t)cols * 4 : orc_row_bytes(fmt, cols);
    if (nx == 0) nx = 1;
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t p = 0; p < nx; ++p)
            y[(size_t)p * ystride + r] += one_dot(fmt, w + r * rb, x + (size_t)p * xstride,
                                                  cols, fast, i8_mask, i8k_mask);
}

typedef struct {
    int fmt; const uint8_t * w; uint32_t r0, r1, cols; const float * x; float * y;
    uint32_t nx, xstride, ystride; int fast; uint32_t i8, i8k;
} mt_job;
static void * mt_run(void * p) {
    mt_job * j = (mt_job *)p;
    const uint64_t rb = j->fmt == ORC_F32 ? (uint64_t)j->cols * 4 : orc_row_bytes(j->fmt, j->cols);
    orc_stream_dot(j->fmt, j->w + j->r0 * rb, j->r1 - j->r0, j->cols, j->x, j->y + j->r0,
                   j->nx, j->xstride, j->ystride, j->fast, j->i8, j->i8k);
    return 0;
}
void orc_stream_dot_mt(int fmt, const uint8_t * w, uint32_t rows, uint32_t cols,
                       const float * x, float * y, uint32_t nx, uint32_t xstride,
                       uint32_t ystride, int fast, uint32_t i8_mask,
                       uint32_t i8k_mask, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if ((uint32_t)nthreads > rows) nthreads = rows ? (int)rows : 1;
    pthread_t * th = (pthread_t *)calloc((size_t)nthreads, sizeof(pthread_t));
    mt_job * jb = (mt_job *)calloc((size_t)nthreads, sizeof(mt_job));
    for (int t = 0; t < nthreads; ++t) {
        mt_job j = { fmt, w, (uint32_t)((uint64_t)rows * t / nthreads),
                     (uint32_t)((uint64_t)rows * (t + 1) / nthreads), cols, x, y,
                     nx, xstride, ystride, fast, i8_mask, i8k_mask };
        jb[t] = j;
        if (t) pthread_create(&th[t], 0, mt_run, &jb[t]);
    }
    mt_run(&jb[0]);
    for (int t = 1; t < nthreads; ++t) pthread_join(th[t], 0);
    free(th); free(jb);
}

/* ---- MoE glue (src/runtime/decode_params.h:234-295) ------------------- */
void orc_router_sel(const float * logits, uint32_t n_expert, uint32_t top_k,
                    uint32_t norm, float scale, uint32_t * ids, float * gates) {
    float mx = -1e30f, sum = 0.f, w[256], tsum = 0.f;
    for (uint32_t i = 0; i < n_expert; ++i) if (logits[i] > mx) mx = logits[i];
    for (uint32_t i = 0; i < n_expert; ++i) { w[i] = expf(logits[i] - mx); sum += w[i]; }
    for (uint32_t i = 0; i < n_expert; ++i) w[i] /= sum;
    for (uint32_t k = 0; k < top_k; ++k) {
        uint32_t best = 0; float bw = -1.f;
        for (uint32_t i = 0; i < n_expert; ++i) {
            int taken = 0;
            for (uint32_t k2 = 0; k2 < k; ++k2) if (ids[k2] == i) { taken = 1; break; }
            if (!taken && w[i] > bw) { bw = w[i]; best = i; }
        }
        ids[k] = best; gates[k] = bw; tsum += bw;
    }
    for (uint32_t k = 0; k < top_k; ++k) {
        if (norm) gates[k] /= tsum;
        gates[k] *= scale;
    }
}
// RMSNORM (src/runtime/decode_params.h:101-106): the sum of squares in
// ascending order, one product and one add per element, each rounded (the
// reference builds with -ffp-contract=off); s = 1 / sqrtf(mean + eps) with a
// correctly rounded sqrtf and division; y = (x * s) * w.
void orc_rmsnorm(const float * wnorm, const float * x, float * y, float eps, uint32_t n) {
    float ss = 0.f;
    for (uint32_t i = 0; i < n; ++i) ss += x[i] * x[i];
    const float s = 1.0f / sqrtf(ss / (float)n + eps);
    for (uint32_t i = 0; i < n; ++i) y[i] = x[i] * s * wnorm[i];
}

void orc_silu_mul(const float * gate, const float * up, float * h, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) { const float g = gate[i]; h[i] = (g / (1.0f + expf(-g))) * up[i]; }
}
void orc_wmerge(const float * parts, const float * gates, const float * add1,
                const float * add2, float * y, float scale, uint32_t n_parts,
                uint32_t n, uint32_t n_full) {
    float gsc = 1.0f;
    if (gates && n_full > n_parts) {
        float s = 0.f, sf = 0.f;
        for (uint32_t q = 0; q < n_parts; ++q) s += gates[q];
        for (uint32_t q = 0; q < n_full; ++q) sf += gates[q];
        if (s > 0.f) gsc = sf / s;
    }
    for (uint32_t i = 0; i < n; ++i) {
        float acc = 0.f;
        for (uint32_t q = 0; q < n_parts; ++q)
            acc += (gates ? gsc * gates[q] : 1.0f) * parts[(size_t)q * n + i];
        acc *= scale;
        if (add1) acc += add1[i];
        if (add2) acc += add2[i];
        y[i] = acc;
    }
}
