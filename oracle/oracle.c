/* CPU oracle of the quantized MUL_MAT path -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Built with gcc -O3 -ffp-contract=off, no -ffast-math, x86-64 baseline ISA (SSE2): every float
 * operation below is a single IEEE binary32 operation in the order written, which is the order of
 * the reference's C++ (cited per function). */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__SSE2__)
#include <emmintrin.h>
#define SGO_SSE2 1
#else
#define SGO_SSE2 0
#endif

enum { SGO_OK = 0, SGO_UNSUPPORTED = 1, SGO_INVALID = 2 };

static uint16_t rd16(const uint8_t * p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

static void wr16(uint8_t * p, uint16_t v) {
    memcpy(p, &v, 2);
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* ---------------------------------------------------------------------------------------------
 * binary16 <-> binary32, round to nearest even (reference src/core/ref/f16.cpp:8-91)
 * ------------------------------------------------------------------------------------------- */

float sgo_half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1Fu) {
        return bits_f32(s | 0x7F800000u | (m << 13)); /* Inf / NaN keep the payload */
    }
    if (e != 0) {
        return bits_f32(s | ((e + 112u) << 23) | (m << 13));
    }
    if (m == 0) {
        return bits_f32(s);
    }
    /* subnormal: shift the leading one up to bit 10 */
    int32_t exp = 113;
    while ((m & 0x400u) == 0) {
        m <<= 1;
        --exp;
    }
    return bits_f32(s | ((uint32_t) exp << 23) | ((m & 0x3FFu) << 13));
}

uint16_t sgo_float_to_half(float f) {
    const uint32_t u = f32_bits(f);
    const uint16_t s = (uint16_t) ((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) {
        /* Inf stays Inf; any NaN becomes the quiet NaN 0x7E00 with the sign kept */
        return (uint16_t) (s | 0x7C00u | (a > 0x7F800000u ? 0x200u : 0u));
    }
    if (a >= 0x477FF000u) {
        /* at or above 65520 = 65504 + half an ulp: rounds to Inf */
        return (uint16_t) (s | 0x7C00u);
    }
    if (a >= 0x38800000u) {
        /* normal half: drop 13 mantissa bits, ties to even; a carry moves into the exponent */
        const uint32_t base = a - 0x38000000u; /* exponent rebased from 127 to 15 */
        const uint32_t keep = base >> 13;
        const uint32_t rest = base & 0x1FFFu;
        const uint32_t up = rest > 0x1000u || (rest == 0x1000u && (keep & 1u));
        return (uint16_t) (s | (keep + up));
    }
    if (a < 0x33000000u) {
        return s; /* below 2^-25: zero (2^-25 exactly ties to the even zero) */
    }
    /* subnormal half: value / 2^-24 rounded to an integer 0..1024, ties to even */
    const uint32_t e = a >> 23;
    const uint32_t sig = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - e; /* 14..24 */
    const uint32_t keep = sig >> shift;
    const uint32_t rest = sig & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1u);
    const uint32_t up = rest > halfway || (rest == halfway && (keep & 1u));
    return (uint16_t) (s | (keep + up)); /* 1024 is the smallest normal, 0x0400 */
}

void sgo_half_to_float_n(const uint16_t * src, float * dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = sgo_half_to_float(src[i]);
}

void sgo_float_to_half_n(const float * src, uint16_t * dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = sgo_float_to_half(src[i]);
}

/* ---------------------------------------------------------------------------------------------
 * block geometry (reference src/tensor/tensor.h:26-52)
 * ------------------------------------------------------------------------------------------- */

size_t sgo_block_size(int32_t dtype) {
    switch (dtype) {
        case SGO_F32:
        case SGO_F16:
        case SGO_BF16: return 1;
        case SGO_Q4_0:
        case SGO_Q8_0: return 32;
        case SGO_Q4_K:
        case SGO_Q6_K: return 256;
        default: return 0;
    }
}

size_t sgo_type_size(int32_t dtype) {
    switch (dtype) {
        case SGO_F32: return 4;
        case SGO_F16:
        case SGO_BF16: return 2;
        case SGO_Q4_0: return 18;
        case SGO_Q8_0: return 34;
        case SGO_Q4_K: return 144;
        case SGO_Q6_K: return 210;
        default: return 0;
    }
}

static int is_quant(int32_t dtype) {
    return dtype == SGO_Q4_0 || dtype == SGO_Q8_0 || dtype == SGO_Q4_K || dtype == SGO_Q6_K;
}

/* ---------------------------------------------------------------------------------------------
 * dequantization (reference src/core/ref/quant.cpp:20-108)
 * ------------------------------------------------------------------------------------------- */

/* 6-bit scale and min of sub-block j of the 12 packed bytes (quant.cpp:20-28) */
static void k4_scale_min(int j, const uint8_t * s, uint8_t * sc, uint8_t * mn) {
    if (j < 4) {
        *sc = (uint8_t) (s[j] & 63);
        *mn = (uint8_t) (s[j + 4] & 63);
    } else {
        *sc = (uint8_t) ((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t) ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* quant.cpp:30-41: element j = ((q & 15) - 8) * d, element j + 16 = ((q >> 4) - 8) * d */
static void deq_q4_0(const uint8_t * src, float * y, int64_t nblocks) {
    for (int64_t b = 0; b < nblocks; ++b, src += 18, y += 32) {
        const float d = sgo_half_to_float(rd16(src));
        for (int j = 0; j < 16; ++j) {
            const int q = src[2 + j];
            y[j] = (float) ((q & 0x0F) - 8) * d;
            y[j + 16] = (float) ((q >> 4) - 8) * d;
        }
    }
}

/* quant.cpp:43-52 */
static void deq_q8_0(const uint8_t * src, float * y, int64_t nblocks) {
    for (int64_t b = 0; b < nblocks; ++b, src += 34, y += 32) {
        const float d = sgo_half_to_float(rd16(src));
        for (int j = 0; j < 32; ++j) y[j] = (float) (int8_t) src[2 + j] * d;
    }
}

/* quant.cpp:54-80: chunk c of 64 elements uses sub-blocks 2c (low nibbles) and 2c+1 (high);
 * y = (d * sc) * q - dmin * m, each product rounded before the subtraction */
static void deq_q4_k(const uint8_t * src, float * y, int64_t nblocks) {
    for (int64_t b = 0; b < nblocks; ++b, src += 144, y += 256) {
        const float d = sgo_half_to_float(rd16(src));
        const float dmin = sgo_half_to_float(rd16(src + 2));
        for (int c = 0; c < 4; ++c) {
            uint8_t sc, mn;
            k4_scale_min(2 * c, src + 4, &sc, &mn);
            const float dlo = d * (float) sc, mlo = dmin * (float) mn;
            k4_scale_min(2 * c + 1, src + 4, &sc, &mn);
            const float dhi = d * (float) sc, mhi = dmin * (float) mn;
            const uint8_t * q = src + 16 + 32 * c;
            for (int l = 0; l < 32; ++l) {
                y[64 * c + l] = dlo * (float) (q[l] & 0x0F) - mlo;
                y[64 * c + 32 + l] = dhi * (float) (q[l] >> 4) - mhi;
            }
        }
    }
}

/* quant.cpp:82-108: half h (128 elements) takes ql[64h..], qh[32h..], scales[8h..]; element
 * 128h + 32r + l (r = 0..3) has 6-bit value (low/high nibble of ql) | (2 bits of qh) << 4, minus 32,
 * times (d * scale[8h + 2r + l/16]) */
static void deq_q6_k(const uint8_t * src, float * y, int64_t nblocks) {
    for (int64_t b = 0; b < nblocks; ++b, src += 210, y += 256) {
        const float d = sgo_half_to_float(rd16(src + 208));
        for (int h = 0; h < 2; ++h) {
            const uint8_t * ql = src + 64 * h;
            const uint8_t * qh = src + 128 + 32 * h;
            const int8_t * sc = (const int8_t *) (src + 192 + 8 * h);
            float * yo = y + 128 * h;
            for (int l = 0; l < 32; ++l) {
                const int s = l / 16;
                const int v0 = ((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32;
                const int v1 = ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int v2 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int v3 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                yo[l] = d * (float) sc[s] * (float) v0;
                yo[l + 32] = d * (float) sc[s + 2] * (float) v1;
                yo[l + 64] = d * (float) sc[s + 4] * (float) v2;
                yo[l + 96] = d * (float) sc[s + 6] * (float) v3;
            }
        }
    }
}

int sgo_dequantize(int32_t dtype, const void * src, float * dst, int64_t n) {
    if (src == NULL || dst == NULL || n <= 0) return SGO_INVALID;
    if (!is_quant(dtype)) return SGO_UNSUPPORTED;
    const int64_t bs = (int64_t) sgo_block_size(dtype);
    if (n % bs != 0) return SGO_INVALID;
    const uint8_t * s = (const uint8_t *) src;
    switch (dtype) {
        case SGO_Q4_0: deq_q4_0(s, dst, n / bs); break;
        case SGO_Q8_0: deq_q8_0(s, dst, n / bs); break;
        case SGO_Q4_K: deq_q4_k(s, dst, n / bs); break;
        default: deq_q6_k(s, dst, n / bs); break;
    }
    return SGO_OK;
}

/* ---------------------------------------------------------------------------------------------
 * quantization (reference src/core/ref/quant.cpp:111-470, ggml's reference quantizers)
 * ------------------------------------------------------------------------------------------- */

/* quant.cpp:111-137 (quantize_row_q4_0_ref): d = (signed value of largest magnitude) / -8 */
static void quant_q4_0(const float * x, uint8_t * dst, int64_t nblocks) {
    for (int64_t b = 0; b < nblocks; ++b, x += 32, dst += 18) {
        float amax = 0.0f, vmax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            if (amax < fabsf(x[j])) {
                amax = fabsf(x[j]);
                vmax = x[j];
            }
        }
        const float d = vmax / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr16(dst, sgo_float_to_half(d));
        for (int j = 0; j < 16; ++j) {
            /* float -> int8 truncation as the reference's static_cast<int8_t>; values are 0.5..16.5 */
            int lo = (int8_t) (int32_t) (x[j] * id + 8.5f);
            int hi = (int8_t) (int32_t) (x[j + 16] * id + 8.5f);
            lo = (uint8_t) lo > 15 ? 15 : (uint8_t) lo;
            hi = (uint8_t) hi > 15 ? 15 : (uint8_t) hi;
            dst[2 + j] = (uint8_t) (lo | (hi << 4));
        }
    }
}

/* quant.cpp:139-159 (quantize_row_q8_0_ref) */
static void quant_q8_0(const float * x, uint8_t * dst, int64_t nblocks) {
    for (int64_t b = 0; b < nblocks; ++b, x += 32, dst += 34) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float a = fabsf(x[j]);
            amax = amax < a ? a : amax;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr16(dst, sgo_float_to_half(d));
        for (int j = 0; j < 32; ++j) dst[2 + j] = (uint8_t) (int8_t) lroundf(x[j] * id);
    }
}

/* quant.cpp:161-166: round to nearest, ties to even, through the 1.5 * 2^23 trick */
static int nearest_int(float v) {
    const uint32_t u = f32_bits(v + 12582912.0f);
    return (int) (u & 0x007FFFFFu) - 0x00400000;
}

static int clampi(int v, int lo, int hi) {
    return v < lo ? lo : v > hi ? hi : v;
}

/* quant.cpp:168-241 (make_qx_quants) specialised to the arguments quantize_row_q6_k passes:
 * n = 16, nmax = 32, rmse_type = 1 (weights x^2), no external weights. Returns the scale; L gets
 * the levels 0..63. */
static float q6_group_scale(const float * x, int8_t * L) {
    const int n = 16, nmax = 32;
    float amax = 0.0f, vmax = 0.0f;
    for (int i = 0; i < n; ++i) {
        if (fabsf(x[i]) > amax) {
            amax = fabsf(x[i]);
            vmax = x[i];
        }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.0f;
    }
    float iscale = -(float) nmax / vmax;
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; ++i) {
        const int l = clampi(nearest_int(iscale * x[i]), -nmax, nmax - 1);
        L[i] = (int8_t) (l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float) l;
        suml2 += w * (float) l * (float) l;
    }
    float scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int step = -9; step <= 9; ++step) {
        if (step == 0) continue;
        iscale = -((float) nmax + 0.1f * (float) step) / vmax;
        sumlx = 0.0f;
        suml2 = 0.0f;
        for (int i = 0; i < n; ++i) {
            const int l = clampi(nearest_int(iscale * x[i]), -nmax, nmax - 1);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * (float) l;
            suml2 += w * (float) l * (float) l;
        }
        if (suml2 > 0.0f && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                L[i] = (int8_t) (nmax + clampi(nearest_int(iscale * x[i]), -nmax, nmax - 1));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

/* quant.cpp:243-325 (make_qkx2_quants) specialised to quantize_row_q4_k's arguments: n = 32,
 * nmax = 15, rmin = -1, rdelta = 0.1, nstep = 20, squared error. Returns the scale, *neg_min = -min. */
static float q4k_group_scale(const float * x, const float * w, uint8_t * L, float * neg_min) {
    const int n = 32, nmax = 15, nstep = 20;
    const float rmin = -1.0f, rdelta = 0.1f;
    uint8_t Laux[32];
    float lo = x[0], hi = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (lo > 0.0f) lo = 0.0f;
    if (hi == lo) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *neg_min = -lo;
        return 0.0f;
    }
    float iscale = (float) nmax / (hi - lo);
    float scale = 1.0f / iscale;
    float best_err = 0.0f;
    for (int i = 0; i < n; ++i) {
        const int l = clampi(nearest_int(iscale * (x[i] - lo)), 0, nmax);
        L[i] = (uint8_t) l;
        const float diff = scale * (float) l + lo - x[i];
        best_err += w[i] * (diff * diff);
    }
    for (int step = 0; step <= nstep; ++step) {
        iscale = (rmin + rdelta * (float) step + (float) nmax) / (hi - lo);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        for (int i = 0; i < n; ++i) {
            const int l = clampi(nearest_int(iscale * (x[i] - lo)), 0, nmax);
            Laux[i] = (uint8_t) l;
            sum_l += w[i] * (float) l;
            sum_l2 += w[i] * (float) l * (float) l;
            sum_xl += w[i] * (float) l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0.0f) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0.0f) {
                this_min = 0.0f;
                this_scale = sum_xl / sum_l2;
            }
            float err = 0.0f;
            for (int i = 0; i < n; ++i) {
                const float diff = this_scale * (float) Laux[i] + this_min - x[i];
                err += w[i] * (diff * diff);
            }
            if (err < best_err) {
                memcpy(L, Laux, (size_t) n);
                best_err = err;
                scale = this_scale;
                lo = this_min;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

/* quant.cpp:327-402 (quantize_row_q4_K_ref) */
static void quant_q4_k(const float * x, uint8_t * dst, int64_t nblocks) {
    uint8_t L[256];
    float w[32], mins[8], scales[8];
    for (int64_t b = 0; b < nblocks; ++b, x += 256, dst += 144) {
        memset(dst, 0, 144);
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; ++j) {
            const float * xs = x + 32 * j;
            float sum_x2 = 0.0f;
            for (int l = 0; l < 32; ++l) sum_x2 += xs[l] * xs[l];
            const float av_x = sqrtf(sum_x2 / 32.0f);
            for (int l = 0; l < 32; ++l) w[l] = av_x + fabsf(xs[l]);
            scales[j] = q4k_group_scale(xs, w, L + 32 * j, &mins[j]);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        uint8_t * s = dst + 4;
        for (int j = 0; j < 8; ++j) {
            uint8_t ls = (uint8_t) nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t) nearest_int(inv_min * mins[j]);
            if (ls > 63) ls = 63;
            if (lm > 63) lm = 63;
            if (j < 4) {
                s[j] = ls;
                s[j + 4] = lm;
            } else {
                s[j + 4] = (uint8_t) ((ls & 0x0F) | ((lm & 0x0F) << 4));
                s[j - 4] = (uint8_t) (s[j - 4] | ((ls >> 4) << 6));
                s[j] = (uint8_t) (s[j] | ((lm >> 4) << 6));
            }
        }
        wr16(dst, sgo_float_to_half(max_scale / 63.0f));
        wr16(dst + 2, sgo_float_to_half(max_min / 63.0f));
        const float dh = sgo_half_to_float(rd16(dst));
        const float mh = sgo_half_to_float(rd16(dst + 2));
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, mn;
            k4_scale_min(j, s, &sc, &mn);
            const float d = dh * (float) sc;
            if (d == 0.0f) continue; /* keeps the levels of the search */
            const float dm = mh * (float) mn;
            for (int i = 0; i < 32; ++i) {
                L[32 * j + i] = (uint8_t) clampi(nearest_int((x[32 * j + i] + dm) / d), 0, 15);
            }
        }
        for (int c = 0; c < 4; ++c) {
            for (int l = 0; l < 32; ++l) {
                dst[16 + 32 * c + l] = (uint8_t) (L[64 * c + l] | (L[64 * c + 32 + l] << 4));
            }
        }
    }
}

/* quant.cpp:404-470 (quantize_row_q6_K_ref) */
static void quant_q6_k(const float * x, uint8_t * dst, int64_t nblocks) {
    int8_t L[256];
    float scales[16];
    for (int64_t b = 0; b < nblocks; ++b, x += 256, dst += 210) {
        float max_scale = 0.0f, max_abs = 0.0f;
        for (int g = 0; g < 16; ++g) {
            scales[g] = q6_group_scale(x + 16 * g, L + 16 * g);
            if (fabsf(scales[g]) > max_abs) {
                max_abs = fabsf(scales[g]);
                max_scale = scales[g];
            }
        }
        if (max_abs < 1e-15f) {
            memset(dst, 0, 210);
            continue;
        }
        const float iscale = -128.0f / max_scale;
        wr16(dst + 208, sgo_float_to_half(1.0f / iscale));
        int8_t * sc = (int8_t *) (dst + 192);
        for (int g = 0; g < 16; ++g) {
            const int v = nearest_int(iscale * scales[g]);
            sc[g] = (int8_t) (v < 127 ? v : 127);
        }
        const float dh = sgo_half_to_float(rd16(dst + 208));
        for (int g = 0; g < 16; ++g) {
            const float d = dh * (float) sc[g];
            if (d == 0.0f) continue;
            for (int i = 0; i < 16; ++i) {
                L[16 * g + i] = (int8_t) (clampi(nearest_int(x[16 * g + i] / d), -32, 31) + 32);
            }
        }
        for (int h = 0; h < 2; ++h) {
            uint8_t * ql = dst + 64 * h;
            uint8_t * qh = dst + 128 + 32 * h;
            const int8_t * Lh = L + 128 * h;
            for (int l = 0; l < 32; ++l) {
                ql[l] = (uint8_t) ((Lh[l] & 0x0F) | ((Lh[l + 64] & 0x0F) << 4));
                ql[l + 32] = (uint8_t) ((Lh[l + 32] & 0x0F) | ((Lh[l + 96] & 0x0F) << 4));
                qh[l] = (uint8_t) ((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) | ((Lh[l + 64] >> 4) << 4) | ((Lh[l + 96] >> 4) << 6));
            }
        }
    }
}

int sgo_quantize(int32_t dtype, const float * src, void * dst, int64_t n) {
    if (src == NULL || dst == NULL || n <= 0) return SGO_INVALID;
    if (!is_quant(dtype)) return SGO_UNSUPPORTED;
    const int64_t bs = (int64_t) sgo_block_size(dtype);
    if (n % bs != 0) return SGO_INVALID;
    uint8_t * d = (uint8_t *) dst;
    switch (dtype) {
        case SGO_Q4_0: quant_q4_0(src, d, n / bs); break;
        case SGO_Q8_0: quant_q8_0(src, d, n / bs); break;
        case SGO_Q4_K: quant_q4_k(src, d, n / bs); break;
        default: quant_q6_k(src, d, n / bs); break;
    }
    return SGO_OK;
}

/* ---------------------------------------------------------------------------------------------
 * MUL_MAT (reference src/core/ref/ops.cpp:802-984)
 *
 * Every output is acc = 0; for k = 0..K-1: acc = acc + (w[k] * x[k]) in float. The reference
 * takes a scalar loop for N < 4 and, for N >= 4, an SSE2 panel of 4/8/16 activation columns laid
 * out K-major; each SIMD lane performs the same increasing-K multiply-then-add, so both give the
 * same bits. The panel is kept here because it is the reference's speed on the CPU baseline.
 * ------------------------------------------------------------------------------------------- */

static const uint8_t * tptr(const sgo_tensor * t, int64_t i1, int64_t i2, int64_t i3) {
    return (const uint8_t *) t->data + (uint64_t) i1 * t->nb[1] + (uint64_t) i2 * t->nb[2] + (uint64_t) i3 * t->nb[3];
}

static int64_t dim(const sgo_tensor * t, int i) {
    return t->ne[i] > 0 ? t->ne[i] : 1;
}

/* a row of src0 as floats (ops.cpp:258-269 with load_float, ops.cpp:32-41,78-93): F16 through
 * half_to_float, BF16 as the high half of an f32, quantized rows dequantized */
static void load_row(const sgo_tensor * w, const uint8_t * p, int64_t K, float * row) {
    if (w->dtype == SGO_F32) {
        memcpy(row, p, (size_t) K * 4);
    } else if (w->dtype == SGO_F16 || w->dtype == SGO_BF16) {
        for (int64_t k = 0; k < K; ++k) {
            uint16_t h;
            memcpy(&h, p + 2 * k, 2);
            if (w->dtype == SGO_F16) {
                row[k] = sgo_half_to_float(h);
            } else {
                const uint32_t bits = (uint32_t) h << 16;
                memcpy(&row[k], &bits, 4);
            }
        }
    } else {
        sgo_dequantize(w->dtype, p, row, K);
    }
}

static int panel_width(int64_t cols) {
    return cols <= 4 ? 4 : cols <= 8 ? 8 : 16;
}

static void panel_dot(const float * row, const float * panel, int64_t K, int width, float * out) {
#if SGO_SSE2
    __m128 acc[4] = {_mm_setzero_ps(), _mm_setzero_ps(), _mm_setzero_ps(), _mm_setzero_ps()};
    const int groups = width / 4;
    for (int64_t k = 0; k < K; ++k) {
        const __m128 a = _mm_set1_ps(row[k]);
        for (int g = 0; g < groups; ++g) {
            acc[g] = _mm_add_ps(acc[g], _mm_mul_ps(a, _mm_loadu_ps(panel + k * width + 4 * g)));
        }
    }
    for (int g = 0; g < groups; ++g) _mm_storeu_ps(out + 4 * g, acc[g]);
#else
    float acc[16] = {0};
    for (int64_t k = 0; k < K; ++k) {
        for (int c = 0; c < width; ++c) acc[c] = acc[c] + row[k] * panel[k * width + c];
    }
    memcpy(out, acc, (size_t) width * 4);
#endif
}

typedef struct mm_job {
    const sgo_tensor * w;
    const sgo_tensor * x;
    sgo_tensor * y;
    int64_t r2, r3;
    int64_t m0, m1; /* rows of every slice handled by this job */
} mm_job;

static void * mm_run(void * arg) {
    const mm_job * j = (const mm_job *) arg;
    const sgo_tensor * w = j->w;
    const sgo_tensor * x = j->x;
    sgo_tensor * y = j->y;
    const int64_t K = dim(w, 0), N = dim(x, 1);
    float * row = (float *) malloc((size_t) K * 4);
    float * panel = N >= 4 ? (float *) malloc((size_t) K * 16 * 4) : NULL;
    for (int64_t i3 = 0; i3 < dim(x, 3); ++i3) {
        for (int64_t i2 = 0; i2 < dim(x, 2); ++i2) {
            const int64_t w2 = i2 / j->r2, w3 = i3 / j->r3;
            if (N >= 4) {
                for (int64_t n0 = 0; n0 < N; n0 += 16) {
                    const int64_t cols = N - n0 < 16 ? N - n0 : 16;
                    const int width = panel_width(cols);
                    for (int64_t k = 0; k < K; ++k) {
                        for (int c = 0; c < width; ++c) {
                            float v = 0.0f;
                            if (c < cols) memcpy(&v, tptr(x, n0 + c, i2, i3) + k * 4, 4);
                            panel[k * width + c] = v;
                        }
                    }
                    for (int64_t m = j->m0; m < j->m1; ++m) {
                        float out[16];
                        load_row(w, tptr(w, m, w2, w3), K, row);
                        panel_dot(row, panel, K, width, out);
                        for (int64_t c = 0; c < cols; ++c) memcpy((uint8_t *) tptr(y, n0 + c, i2, i3) + m * 4, &out[c], 4);
                    }
                }
            } else {
                for (int64_t m = j->m0; m < j->m1; ++m) {
                    load_row(w, tptr(w, m, w2, w3), K, row);
                    for (int64_t n = 0; n < N; ++n) {
                        const float * xv = (const float *) tptr(x, n, i2, i3);
                        float acc = 0.0f;
                        for (int64_t k = 0; k < K; ++k) acc = acc + row[k] * xv[k];
                        memcpy((uint8_t *) tptr(y, n, i2, i3) + m * 4, &acc, 4);
                    }
                }
            }
        }
    }
    free(row);
    free(panel);
    return NULL;
}

/* the checks of exec_mul_mat (ops.cpp:891-920) */
static int mm_check(const sgo_tensor * w, const sgo_tensor * x, const sgo_tensor * y, int allow_broadcast, int64_t * r2, int64_t * r3) {
    if (w == NULL || x == NULL || y == NULL || w->data == NULL || x->data == NULL || y->data == NULL) return SGO_INVALID;
    if (x->dtype != SGO_F32 || y->dtype != SGO_F32) return SGO_UNSUPPORTED;
    if (w->dtype != SGO_F32 && w->dtype != SGO_F16 && w->dtype != SGO_BF16 && !is_quant(w->dtype)) return SGO_UNSUPPORTED;
    if (w->nb[0] != sgo_type_size(w->dtype)) return SGO_UNSUPPORTED;
    if (is_quant(w->dtype) && dim(w, 0) % (int64_t) sgo_block_size(w->dtype) != 0) return SGO_UNSUPPORTED;
    if (dim(w, 0) != dim(x, 0)) return SGO_INVALID;
    if (x->nb[0] != 4 || y->nb[0] != 4) return SGO_UNSUPPORTED;
    if (dim(x, 2) % dim(w, 2) != 0 || dim(x, 3) % dim(w, 3) != 0) return SGO_INVALID;
    *r2 = dim(x, 2) / dim(w, 2);
    *r3 = dim(x, 3) / dim(w, 3);
    if (!allow_broadcast && (*r2 != 1 || *r3 != 1)) return SGO_UNSUPPORTED;
    if (dim(y, 0) != dim(w, 1) || dim(y, 1) != dim(x, 1) || dim(y, 2) != dim(x, 2) || dim(y, 3) != dim(x, 3)) return SGO_INVALID;
    return SGO_OK;
}

int sgo_mul_mat(const sgo_tensor * w, const sgo_tensor * x, sgo_tensor * y, int allow_broadcast) {
    return sgo_mul_mat_mt(w, x, y, allow_broadcast, 1);
}

int sgo_mul_mat_mt(const sgo_tensor * w, const sgo_tensor * x, sgo_tensor * y, int allow_broadcast, int threads) {
    int64_t r2 = 1, r3 = 1;
    const int st = mm_check(w, x, y, allow_broadcast, &r2, &r3);
    if (st != SGO_OK) return st;
    const int64_t M = dim(w, 1);
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if ((int64_t) threads > M) threads = (int) M;
    mm_job jobs[256];
    pthread_t tids[256];
    for (int t = 0; t < threads; ++t) {
        jobs[t].w = w;
        jobs[t].x = x;
        jobs[t].y = y;
        jobs[t].r2 = r2;
        jobs[t].r3 = r3;
        jobs[t].m0 = M * t / threads;
        jobs[t].m1 = M * (t + 1) / threads;
    }
    if (threads == 1) {
        mm_run(&jobs[0]);
        return SGO_OK;
    }
    for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, mm_run, &jobs[t]);
    for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    return SGO_OK;
}

/* ---------------------------------------------------------------------------------------------
 * MUL_MAT_ID (reference src/core/ref/ops.cpp:986-1024): expert matrices w [K, M, E], activations
 * x [K, n1, T] (n1 = 1: shared by the slots, or n1 = n_used), ids I32 [n_used, T], dst
 * [M, n_used, T]: dst[:, i, t] = w[:, :, ids[i, t]] x[:, i or 0, t]. Every output is the scalar
 * increasing-K loop of MUL_MAT at one column; an expert index outside [0, E) is an error, found
 * in (t, i) order (outputs of earlier pairs stay written, as in the reference).
 * ------------------------------------------------------------------------------------------- */

static int ids_i32(const sgo_tensor * ids, int64_t i, int64_t t, int32_t * e) {
    memcpy(e, (const uint8_t *) ids->data + (uint64_t) i * ids->nb[0] + (uint64_t) t * ids->nb[1], 4);
    return SGO_OK;
}

int sgo_mul_mat_id(const sgo_tensor * w, const sgo_tensor * x, const sgo_tensor * ids, sgo_tensor * y) {
    if (w == NULL || x == NULL || ids == NULL || y == NULL || w->data == NULL || x->data == NULL || ids->data == NULL || y->data == NULL) return SGO_INVALID;
    if (x->dtype != SGO_F32 || y->dtype != SGO_F32 || ids->dtype != SGO_I32) return SGO_UNSUPPORTED;
    if (w->dtype != SGO_F32 && w->dtype != SGO_F16 && !is_quant(w->dtype)) return SGO_UNSUPPORTED;
    if (w->nb[0] != sgo_type_size(w->dtype)) return SGO_UNSUPPORTED;
    if (dim(w, 3) != 1 || dim(x, 3) != 1 || dim(ids, 2) != 1 || dim(ids, 3) != 1) return SGO_INVALID;
    if (dim(w, 0) != dim(x, 0) || (dim(x, 1) != 1 && dim(x, 1) != dim(ids, 0)) || dim(x, 2) != dim(ids, 1) ||
        dim(y, 0) != dim(w, 1) || dim(y, 1) != dim(ids, 0) || dim(y, 2) != dim(ids, 1) || dim(y, 3) != 1) {
        return SGO_INVALID;
    }
    const int64_t K = dim(w, 0), M = dim(w, 1), E = dim(w, 2);
    if (is_quant(w->dtype) && K % (int64_t) sgo_block_size(w->dtype) != 0) return SGO_UNSUPPORTED;
    float * row = (float *) malloc((size_t) K * 4);
    for (int64_t t = 0; t < dim(ids, 1); ++t) {
        for (int64_t i = 0; i < dim(ids, 0); ++i) {
            int32_t e;
            ids_i32(ids, i, t, &e);
            if (e < 0 || (int64_t) e >= E) {
                free(row);
                return SGO_INVALID;
            }
            const int64_t i11 = dim(x, 1) == 1 ? 0 : i;
            const float * xv = (const float *) tptr(x, i11, t, 0);
            for (int64_t m = 0; m < M; ++m) {
                load_row(w, tptr(w, m, e, 0), K, row);
                float acc = 0.0f;
                for (int64_t k = 0; k < K; ++k) acc = acc + row[k] * xv[k];
                memcpy((uint8_t *) tptr(y, i, t, 0) + m * 4, &acc, 4);
            }
        }
    }
    free(row);
    return SGO_OK;
}

/* ---------------------------------------------------------------------------------------------
 * GET_ROWS (reference src/core/ref/ops.cpp:690-721): src0 [K, R, S2, S3] (rows of K elements),
 * ids I32 [n, i11 < S2, i12 < S3], dst F32 [K, n, ids ne1, ids ne2]: dst[:, a, b, c] = row
 * ids[a, b, c] of slice (b, c) of src0, dequantized. A row index outside [0, R) is an error,
 * found in (c, b, a) order.
 * ------------------------------------------------------------------------------------------- */

int sgo_get_rows(const sgo_tensor * w, const sgo_tensor * ids, sgo_tensor * y) {
    if (w == NULL || ids == NULL || y == NULL || w->data == NULL || ids->data == NULL || y->data == NULL) return SGO_INVALID;
    if (ids->dtype != SGO_I32 || y->dtype != SGO_F32) return SGO_UNSUPPORTED;
    if (w->dtype != SGO_F32 && w->dtype != SGO_F16 && !is_quant(w->dtype)) return SGO_UNSUPPORTED;
    if (w->nb[0] != sgo_type_size(w->dtype)) return SGO_UNSUPPORTED;
    if (dim(ids, 3) != 1 || dim(ids, 1) > dim(w, 2) || dim(ids, 2) > dim(w, 3) || dim(y, 0) != dim(w, 0) || dim(y, 1) != dim(ids, 0) ||
        dim(y, 2) != dim(ids, 1) || dim(y, 3) != dim(ids, 2)) {
        return SGO_INVALID;
    }
    const int64_t K = dim(w, 0);
    if (is_quant(w->dtype) && K % (int64_t) sgo_block_size(w->dtype) != 0) return SGO_UNSUPPORTED;
    float * row = (float *) malloc((size_t) K * 4);
    for (int64_t c = 0; c < dim(ids, 2); ++c) {
        for (int64_t b = 0; b < dim(ids, 1); ++b) {
            for (int64_t a = 0; a < dim(ids, 0); ++a) {
                int32_t r;
                memcpy(&r, (const uint8_t *) ids->data + (uint64_t) a * ids->nb[0] + (uint64_t) b * ids->nb[1] + (uint64_t) c * ids->nb[2], 4);
                if (r < 0 || (int64_t) r >= dim(w, 1)) {
                    free(row);
                    return SGO_INVALID;
                }
                load_row(w, tptr(w, r, b, c), K, row);
                uint8_t * out = (uint8_t *) y->data + (uint64_t) a * y->nb[1] + (uint64_t) b * y->nb[2] + (uint64_t) c * y->nb[3];
                for (int64_t k = 0; k < K; ++k) memcpy(out + (uint64_t) k * y->nb[0], &row[k], 4);
            }
        }
    }
    free(row);
    return SGO_OK;
}

/* ---------------------------------------------------------------------------------------------
 * R32 (reference src/tensor/tensor.cpp:5-19, src/backends/opencl11/r32.h:35-90)
 *
 * Per slice of M rows and nb blocks per row, the bytes of a block are split into areas stored one
 * after the other; area k starts at M * nb * (bytes per block of the earlier areas). Rows are
 * grouped by 32 (rs rows in the last group). In an area of 16 * U bytes per block, group g starts
 * at g * 32 * nb * 16U and 16-byte unit j of block b of row `lane` sits at unit (b*U + j)*rs + lane;
 * an area of 2 bytes is an array of halves at b * rs + lane.
 * ------------------------------------------------------------------------------------------- */

typedef struct r32_area_t {
    int src, len;
    uint8_t xr;
} r32_area_t;

static int r32_areas(int32_t dtype, r32_area_t * a) {
    switch (dtype) {
        case SGO_Q8_0: a[0] = (r32_area_t){2, 32, 0x80}; a[1] = (r32_area_t){0, 2, 0}; return 2;
        case SGO_Q4_0: a[0] = (r32_area_t){2, 16, 0}; a[1] = (r32_area_t){0, 2, 0}; return 2;
        case SGO_Q4_K: a[0] = (r32_area_t){16, 128, 0}; a[1] = (r32_area_t){0, 16, 0}; return 2;
        case SGO_Q6_K: a[0] = (r32_area_t){0, 192, 0}; a[1] = (r32_area_t){192, 16, 0x80}; a[2] = (r32_area_t){208, 2, 0}; return 3;
        default: return 0;
    }
}

static int r32_move(int32_t dtype, int64_t K, int64_t M, int64_t slices, uint8_t * nat, uint8_t * rep, int pack) {
    r32_area_t A[3];
    const int na = r32_areas(dtype, A);
    if (na == 0) return SGO_UNSUPPORTED;
    if (K <= 0 || M <= 0 || slices <= 0 || K % (int64_t) sgo_block_size(dtype) != 0) return SGO_INVALID;
    const int64_t nb = K / (int64_t) sgo_block_size(dtype);
    const size_t bs = sgo_type_size(dtype);
    const size_t rowb = (size_t) nb * bs;
    for (int64_t s = 0; s < slices; ++s) {
        uint8_t * ns = nat + (size_t) s * (size_t) M * rowb;
        uint8_t * rs_ = rep + (size_t) s * (size_t) M * rowb;
        size_t before = 0;
        for (int k = 0; k < na; ++k) {
            uint8_t * area = rs_ + (size_t) M * (size_t) nb * before;
            const int U = A[k].len / 16;
            for (int64_t g0 = 0; g0 < M; g0 += 32) {
                const int64_t rs = M - g0 < 32 ? M - g0 : 32;
                uint8_t * grp = area + (size_t) (g0 / 32) * 32 * (size_t) nb * (size_t) A[k].len;
                for (int64_t lane = 0; lane < rs; ++lane) {
                    for (int64_t b = 0; b < nb; ++b) {
                        uint8_t * p = ns + (size_t) (g0 + lane) * rowb + (size_t) b * bs + (size_t) A[k].src;
                        if (A[k].len == 2) {
                            uint8_t * q = grp + ((size_t) b * (size_t) rs + (size_t) lane) * 2;
                            if (pack) memcpy(q, p, 2); else memcpy(p, q, 2);
                            continue;
                        }
                        for (int j = 0; j < U; ++j) {
                            uint8_t * q = grp + (((size_t) b * (size_t) U + (size_t) j) * (size_t) rs + (size_t) lane) * 16;
                            for (int i = 0; i < 16; ++i) {
                                if (pack) q[i] = (uint8_t) (p[16 * j + i] ^ A[k].xr);
                                else p[16 * j + i] = (uint8_t) (q[i] ^ A[k].xr);
                            }
                        }
                    }
                }
            }
            before += (size_t) A[k].len;
        }
    }
    return SGO_OK;
}

int sgo_r32_pack(int32_t dtype, int64_t K, int64_t M, int64_t slices, const uint8_t * nat, uint8_t * rep) {
    if (nat == NULL || rep == NULL) return SGO_INVALID;
    return r32_move(dtype, K, M, slices, (uint8_t *) nat, rep, 1);
}

int sgo_r32_unpack(int32_t dtype, int64_t K, int64_t M, int64_t slices, const uint8_t * rep, uint8_t * nat) {
    if (nat == NULL || rep == NULL) return SGO_INVALID;
    return r32_move(dtype, K, M, slices, nat, (uint8_t *) rep, 0);
}
