// Weight-format kernels of the upload path: R32 pack / unpack in HBM, bit-exact dequantization,
// reference-identical quantization and the synthetic normal generator.
//
// Compiled with -ffp-contract=off (and the pragma below): the quantizer and the dequantizer must
// perform one IEEE binary32 operation per source operation, in the order of the reference's
// src/core/ref/quant.cpp, to reproduce its bytes and floats exactly. Division and sqrt are the
// correctly rounded ones (HIP's default for fp32).
#pragma clang fp contract(off)

#include "kernels.h"

#include <hip/hip_fp16.h>

#include <cmath>

namespace sgk {

Areas areas_of(int dtype) {
    switch (dtype) {
        case Q8_0: return Areas{2, {2, 0, 0}, {32, 2, 0}, {0x80, 0, 0}};
        case Q4_0: return Areas{2, {2, 0, 0}, {16, 2, 0}, {0, 0, 0}};
        case Q4_K: return Areas{2, {16, 0, 0}, {128, 16, 0}, {0, 0, 0}};
        case Q6_K: return Areas{3, {0, 192, 208}, {192, 16, 2}, {0, 0x80, 0}};
        default: return Areas{0, {0, 0, 0}, {0, 0, 0}, {0, 0, 0}};
    }
}

namespace {

int block_elems(int dt) {
    return dt == Q4_K || dt == Q6_K ? 256 : 32;
}

int block_bytes(int dt) {
    switch (dt) {
        case Q4_0: return 18;
        case Q8_0: return 34;
        case Q4_K: return 144;
        default: return 210;
    }
}

// ---- R32 ----------------------------------------------------------------------------------------
// One thread per 16-byte unit (or 2-byte half) of one area. blockIdx.y is the row group inside the
// chunk; the index inside a group runs over units u = b * U + j (slow) and lanes (fast), so that
// consecutive threads write consecutive R32 bytes.
struct MoveArgs {
    uint8_t * nat;     // natural bytes of rows [row0, row0 + nrows)
    uint8_t * area;    // R32 base of this area in the slice
    int64_t M, nb, row0, nrows;
    int bs, src, len;
    uint8_t xr;
    int pack;
};

__global__ __launch_bounds__(256) void k_r32_move(MoveArgs a) {
    const int64_t g0 = a.row0 + 32 * (int64_t) blockIdx.y; // first row of the group (slice row)
    const int rs = (int) min<int64_t>(32, a.M - g0);
    const int U = a.len == 2 ? 1 : a.len / 16;
    const int64_t per_group = 32 * a.nb * U;
    uint8_t * grp = a.area + (uint64_t) g0 * a.nb * a.len;
    for (int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; t < per_group; t += (int64_t) gridDim.x * blockDim.x) {
        const int lane = (int) (t & 31);
        const int64_t u = t >> 5;
        if (lane >= rs) continue;
        const int64_t b = u / U;
        const int j = (int) (u - b * U);
        uint8_t * p = a.nat + (uint64_t) (g0 - a.row0 + lane) * a.nb * a.bs + (uint64_t) b * a.bs + a.src;
        if (a.len == 2) {
            uint16_t * q = reinterpret_cast<uint16_t *>(grp + ((uint64_t) b * rs + lane) * 2);
            uint16_t * pn = reinterpret_cast<uint16_t *>(p); // natural blocks are 2-byte aligned
            if (a.pack) *q = *pn; else *pn = *q;
            continue;
        }
        uint8_t * q = grp + (((uint64_t) u) * rs + lane) * 16;
        uint16_t * pn = reinterpret_cast<uint16_t *>(p + 16 * j);
        const uint32_t x2 = (uint32_t) a.xr * 0x0101u;
        if (a.pack) {
            uint32_t w[4];
            for (int i = 0; i < 4; ++i) w[i] = ((uint32_t) pn[2 * i] | ((uint32_t) pn[2 * i + 1] << 16)) ^ (x2 * 0x00010001u);
            *reinterpret_cast<uint4 *>(q) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            const uint4 v = *reinterpret_cast<const uint4 *>(q);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            for (int i = 0; i < 4; ++i) {
                const uint32_t o = w[i] ^ (x2 * 0x00010001u);
                pn[2 * i] = (uint16_t) (o & 0xFFFFu);
                pn[2 * i + 1] = (uint16_t) (o >> 16);
            }
        }
    }
}

// ---- binary16 <-> binary32 (same rules as the reference's src/core/ref/f16.cpp) ----------------

__device__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

__device__ uint16_t f2h(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint16_t s = (uint16_t) ((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t) (s | 0x7C00u | (a > 0x7F800000u ? 0x200u : 0u));
    if (a >= 0x477FF000u) return (uint16_t) (s | 0x7C00u);
    if (a >= 0x38800000u) {
        const uint32_t base = a - 0x38000000u;
        const uint32_t keep = base >> 13, rest = base & 0x1FFFu;
        return (uint16_t) (s | (keep + (rest > 0x1000u || (rest == 0x1000u && (keep & 1u)))));
    }
    if (a < 0x33000000u) return s;
    const uint32_t shift = 126u - (a >> 23);
    const uint32_t sig = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t keep = sig >> shift, rest = sig & ((1u << shift) - 1u), halfway = 1u << (shift - 1u);
    return (uint16_t) (s | (keep + (rest > halfway || (rest == halfway && (keep & 1u)))));
}

__device__ uint16_t rd16(const uint8_t * p) {
    return (uint16_t) (p[0] | (p[1] << 8));
}

__device__ void wr16(uint8_t * p, uint16_t v) {
    p[0] = (uint8_t) (v & 0xFF);
    p[1] = (uint8_t) (v >> 8);
}

__device__ void k4_scale_min(int j, const uint8_t * s, uint8_t * sc, uint8_t * mn) {
    if (j < 4) {
        *sc = (uint8_t) (s[j] & 63);
        *mn = (uint8_t) (s[j + 4] & 63);
    } else {
        *sc = (uint8_t) ((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t) ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

// ---- dequantization: one thread per output element -------------------------------------------

// element i of the natural block at blk (the reference's dequantize_row_* formulas, quant.cpp:30-108)
template <int DT>
__device__ __forceinline__ float deq_elem(const uint8_t * blk, int i) {
    if (DT == Q4_0) {
        const float d = h2f(rd16(blk));
        const int q = blk[2 + (i & 15)];
        return (float) ((i < 16 ? (q & 0x0F) : (q >> 4)) - 8) * d;
    } else if (DT == Q8_0) {
        return (float) (int8_t) blk[2 + i] * h2f(rd16(blk));
    } else if (DT == Q4_K) {
        const int c = i / 64, l = i % 32, hi = (i % 64) >= 32;
        uint8_t sc, mn;
        k4_scale_min(2 * c + hi, blk + 4, &sc, &mn);
        const float d1 = h2f(rd16(blk)) * (float) sc;
        const float m1 = h2f(rd16(blk + 2)) * (float) mn;
        const int q = blk[16 + 32 * c + l];
        return d1 * (float) (hi ? (q >> 4) : (q & 0x0F)) - m1;
    } else {
        const int h = i / 128, r = (i % 128) / 32, l = i % 32;
        const uint8_t * ql = blk + 64 * h;
        const uint8_t qh = blk[128 + 32 * h + l];
        const int lowq = (r & 1) ? ql[l + 32] : ql[l];
        const int nib = r < 2 ? (lowq & 0x0F) : (lowq >> 4);
        const int v = (nib | (((qh >> (2 * r)) & 3) << 4)) - 32;
        const int8_t sc = (int8_t) blk[192 + 8 * h + 2 * r + l / 16];
        return h2f(rd16(blk + 208)) * (float) sc * (float) v;
    }
}

template <int DT>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t * src, float * dst, int64_t n) {
    constexpr int BS = DT == Q4_K || DT == Q6_K ? 256 : 32;
    constexpr int BB = DT == Q4_0 ? 18 : DT == Q8_0 ? 34 : DT == Q4_K ? 144 : 210;
    for (int64_t e = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t) gridDim.x * blockDim.x) {
        dst[e] = deq_elem<DT>(src + (e / BS) * BB, (int) (e % BS));
    }
}

// ---- quantization: one thread per block (the reference's ggml quantizers) --------------------

__device__ int nearest_int(float v) {
    return (int) (__float_as_uint(v + 12582912.0f) & 0x007FFFFFu) - 0x00400000;
}

__device__ int clampi(int v, int lo, int hi) {
    return v < lo ? lo : v > hi ? hi : v;
}

__device__ void quant_q4_0(const float * x, uint8_t * dst) {
    float amax = 0.0f, vmax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        if (amax < fabsf(x[j])) {
            amax = fabsf(x[j]);
            vmax = x[j];
        }
    }
    const float d = vmax / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    wr16(dst, f2h(d));
    for (int j = 0; j < 16; ++j) {
        int lo = (int8_t) (int32_t) (x[j] * id + 8.5f);
        int hi = (int8_t) (int32_t) (x[j + 16] * id + 8.5f);
        lo = (uint8_t) lo > 15 ? 15 : (uint8_t) lo;
        hi = (uint8_t) hi > 15 ? 15 : (uint8_t) hi;
        dst[2 + j] = (uint8_t) (lo | (hi << 4));
    }
}

__device__ void quant_q8_0(const float * x, uint8_t * dst) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        const float a = fabsf(x[j]);
        amax = amax < a ? a : amax;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    wr16(dst, f2h(d));
    for (int j = 0; j < 32; ++j) dst[2 + j] = (uint8_t) (int8_t) lroundf(x[j] * id);
}

__device__ float q6_group_scale(const float * x, int8_t * L) {
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
            for (int i = 0; i < n; ++i) L[i] = (int8_t) (nmax + clampi(nearest_int(iscale * x[i]), -nmax, nmax - 1));
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

__device__ float q4k_group_scale(const float * x, const float * w, uint8_t * L, float * neg_min) {
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
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_err = err;
                scale = this_scale;
                lo = this_min;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

__device__ void quant_q4_k(const float * x, uint8_t * dst) {
    uint8_t L[256];
    float w[32], mins[8], scales[8];
    for (int i = 0; i < 144; ++i) dst[i] = 0;
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
    wr16(dst, f2h(max_scale / 63.0f));
    wr16(dst + 2, f2h(max_min / 63.0f));
    const float dh = h2f(rd16(dst)), mh = h2f(rd16(dst + 2));
    for (int j = 0; j < 8; ++j) {
        uint8_t sc, mn;
        k4_scale_min(j, s, &sc, &mn);
        const float d = dh * (float) sc;
        if (d == 0.0f) continue;
        const float dm = mh * (float) mn;
        for (int i = 0; i < 32; ++i) L[32 * j + i] = (uint8_t) clampi(nearest_int((x[32 * j + i] + dm) / d), 0, 15);
    }
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l) dst[16 + 32 * c + l] = (uint8_t) (L[64 * c + l] | (L[64 * c + 32 + l] << 4));
}

__device__ void quant_q6_k(const float * x, uint8_t * dst) {
    int8_t L[256];
    float scales[16];
    float max_scale = 0.0f, max_abs = 0.0f;
    for (int g = 0; g < 16; ++g) {
        scales[g] = q6_group_scale(x + 16 * g, L + 16 * g);
        if (fabsf(scales[g]) > max_abs) {
            max_abs = fabsf(scales[g]);
            max_scale = scales[g];
        }
    }
    if (max_abs < 1e-15f) {
        for (int i = 0; i < 210; ++i) dst[i] = 0;
        return;
    }
    const float iscale = -128.0f / max_scale;
    wr16(dst + 208, f2h(1.0f / iscale));
    int8_t * sc = reinterpret_cast<int8_t *>(dst + 192);
    for (int g = 0; g < 16; ++g) {
        const int v = nearest_int(iscale * scales[g]);
        sc[g] = (int8_t) (v < 127 ? v : 127);
    }
    const float dh = h2f(rd16(dst + 208));
    for (int g = 0; g < 16; ++g) {
        const float d = dh * (float) sc[g];
        if (d == 0.0f) continue;
        for (int i = 0; i < 16; ++i) L[16 * g + i] = (int8_t) (clampi(nearest_int(x[16 * g + i] / d), -32, 31) + 32);
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

template <int DT>
__global__ __launch_bounds__(128) void k_quant(const float * src, uint8_t * dst, int64_t nblocks) {
    const int64_t b = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    if (DT == Q4_0) quant_q4_0(src + 32 * b, dst + 18 * b);
    if (DT == Q8_0) quant_q8_0(src + 32 * b, dst + 34 * b);
    if (DT == Q4_K) quant_q4_k(src + 256 * b, dst + 144 * b);
    if (DT == Q6_K) quant_q6_k(src + 256 * b, dst + 210 * b);
}

// ---- synthetic normals: splitmix64(seed, i) -> two 53-bit uniforms -> Box-Muller ---------------

__device__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void k_fill_normal(float * dst, int64_t n, uint64_t seed, float mean, float stddev) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        const uint64_t a = splitmix64(seed * 0xD1B54A32D192ED03ull + 2 * (uint64_t) i);
        const uint64_t b = splitmix64(seed * 0xD1B54A32D192ED03ull + 2 * (uint64_t) i + 1);
        const double u1 = ((double) (a >> 11) + 1.0) * (1.0 / 9007199254740993.0); // (0, 1]
        const double u2 = (double) (b >> 11) * (1.0 / 9007199254740992.0);
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        dst[i] = (float) (mean + stddev * z);
    }
}

// ---- GET_ROWS on R32 weights: one work-group per output row ------------------------------------
// Byte j of natural block b of the selected row is read where the R32 layout put it (the areas of
// areas_of(): area k of the slice at M * nb * (bytes per block of the earlier areas); inside an
// area of L bytes per block, group g0 starts at g0 * nb * L and 16-byte unit u of block b of row
// `lane` sits at ((b * L / 16 + u) * rs + lane) * 16; a 2-byte area is an array of halves at
// (b * rs + lane) * 2), and the element formulas are those of k_dequant (bit-exact).
struct GetRowsArgs {
    const uint8_t * w;    // slice (0, 0) of src0
    uint64_t w_s2, w_s3;  // slice strides (bytes)
    const int32_t * ids;
    int64_t i_s0, i_s1, i_s2; // element strides of ids
    float * y;
    int64_t y_s1, y_s2, y_s3; // element strides of dst
    int64_t K, M, nb, n0, n1; // n0, n1: ids ne0, ne1 (rows = n0 * n1 * ne2)
};

// the row's natural bytes are staged in LDS, kGetRowsBlocks blocks at a time: each R32 unit of the
// row (16 bytes at ((b U + u) rs + lane) 16 of its area, or a 2-byte half at (b rs + lane) 2) is
// one load, all of a pass issued before any is used; then every element is dequantized from LDS
// with the dequantizer's formula
constexpr int kGetRowsBlocks = 64;

// one pass of GET_ROWS over blocks b0 .. b0 + nblk - 1 of one row: the slice, M nb (the bytes
// per block of an area multiply it to give the area's start), g0 nb, rows in the group, the row's
// place in it
struct GrPass {
    const uint8_t * slice;
    uint64_t mnb, g0nb, rs, lane;
    int64_t b0;
    int nblk;
};

// area K of format DT's R32 layout (areas_of, as compile-time constants): at byte BEFORE x M nb
// of the slice, LEN bytes per block, at natural offset SRC, stored xor XR; K past the format's
// areas does nothing. load() fetches the thread's units of the pass into registers (16-byte
// units: at most kGetRowsBlocks x 12 / 256 = 3 per thread; 2-byte halves: one), scatter() puts
// their bytes at their natural places in LDS.
template <int DT, int K>
struct GrArea {
    static constexpr int NA = DT == Q6_K ? 3 : 2;
    static constexpr int SRC = K == 0 ? (DT == Q6_K ? 0 : DT == Q4_K ? 16 : 2) : K == 1 ? (DT == Q6_K ? 192 : 0) : 208;
    static constexpr int LEN = K == 0 ? (DT == Q6_K ? 192 : DT == Q4_K ? 128 : DT == Q8_0 ? 32 : 16) : K == 1 ? (DT == Q6_K || DT == Q4_K ? 16 : 2) : 2;
    static constexpr int BEFORE = K == 0 ? 0 : K == 1 ? (DT == Q6_K ? 192 : DT == Q4_K ? 128 : DT == Q8_0 ? 32 : 16) : 208;
    static constexpr uint32_t XR = (K == 0 && DT == Q8_0) || (K == 1 && DT == Q6_K) ? 0x80u : 0u;
    static constexpr int U = LEN / 16, NU = U > 0 ? (kGetRowsBlocks * U + 255) / 256 : 1;
    uint4 v[NU];
    uint32_t hv;
    __device__ void load(const GrPass & p) {
        if constexpr (K < NA) {
            const uint8_t * area = p.slice + p.mnb * BEFORE;
            if constexpr (LEN == 2) {
                const int t = threadIdx.x;
                hv = t < p.nblk ? (uint32_t) *reinterpret_cast<const uint16_t *>(area + p.g0nb * 2 + ((uint64_t) (p.b0 + t) * p.rs + p.lane) * 2) : 0u;
            } else {
#pragma unroll
                for (int i = 0; i < NU; ++i) {
                    const int t = threadIdx.x + 256 * i, bl = t / U, u = t - bl * U;
                    if (t < p.nblk * U) v[i] = *reinterpret_cast<const uint4 *>(area + p.g0nb * LEN + (((uint64_t) (p.b0 + bl) * U + u) * p.rs + p.lane) * 16);
                }
            }
        }
    }
    __device__ void scatter(const GrPass & p, uint8_t * nat, int bb) const {
        if constexpr (K < NA) {
            if constexpr (LEN == 2) {
                const int t = threadIdx.x;
                if (t < p.nblk) {
                    nat[t * bb + SRC] = (uint8_t) (hv & 0xFFu);
                    nat[t * bb + SRC + 1] = (uint8_t) (hv >> 8);
                }
            } else {
#pragma unroll
                for (int i = 0; i < NU; ++i) {
                    const int t = threadIdx.x + 256 * i, bl = t / U, u = t - bl * U;
                    if (t < p.nblk * U) {
                        const uint32_t m = XR * 0x01010101u;
                        const uint32_t w[4] = {v[i].x ^ m, v[i].y ^ m, v[i].z ^ m, v[i].w ^ m};
                        uint8_t * d = nat + bl * bb + SRC + 16 * u; // natural offsets are not 4-aligned in general
                        for (int q = 0; q < 16; ++q) d[q] = (uint8_t) (w[q >> 2] >> (8 * (q & 3)));
                    }
                }
            }
        }
    }
};

// the kernel's compile-time areas against areas_of() (the layout the weights were packed in)
template <int DT>
bool gr_areas_match() {
    const Areas ar = areas_of(DT);
    const int src[3] = {GrArea<DT, 0>::SRC, GrArea<DT, 1>::SRC, GrArea<DT, 2>::SRC};
    const int len[3] = {GrArea<DT, 0>::LEN, GrArea<DT, 1>::LEN, GrArea<DT, 2>::LEN};
    const uint32_t xr[3] = {GrArea<DT, 0>::XR, GrArea<DT, 1>::XR, GrArea<DT, 2>::XR};
    if (ar.na != GrArea<DT, 0>::NA) return false;
    int before = 0;
    for (int k = 0; k < ar.na; ++k) {
        const int bk = k == 0 ? GrArea<DT, 0>::BEFORE : k == 1 ? GrArea<DT, 1>::BEFORE : GrArea<DT, 2>::BEFORE;
        if (ar.src[k] != src[k] || ar.len[k] != len[k] || ar.xr[k] != xr[k] || bk != before) return false;
        before += ar.len[k];
    }
    return true;
}

template <int DT>
__global__ __launch_bounds__(256) void k_get_rows(GetRowsArgs a) {
    constexpr int BS = DT == Q4_K || DT == Q6_K ? 256 : 32;
    constexpr int BB = DT == Q4_0 ? 18 : DT == Q8_0 ? 34 : DT == Q4_K ? 144 : 210;
    __shared__ __attribute__((aligned(16))) uint8_t nat[kGetRowsBlocks * BB];
    const int64_t row = blockIdx.x;
    const int64_t c = row / (a.n0 * a.n1), rem = row - c * a.n0 * a.n1, bi = rem / a.n0, ai = rem - bi * a.n0;
    int64_t r = a.ids[ai * a.i_s0 + bi * a.i_s1 + c * a.i_s2];
    r = r < 0 ? 0 : (r >= a.M ? a.M - 1 : r); // out-of-range rows read the nearest row
    const uint8_t * slice = a.w + (uint64_t) bi * a.w_s2 + (uint64_t) c * a.w_s3;
    const int64_t g0 = r & ~(int64_t) 31;
    const int64_t rs = a.M - g0 < 32 ? a.M - g0 : 32, lane = r - g0;
    float * y = a.y + ai * a.y_s1 + bi * a.y_s2 + c * a.y_s3;
    for (int64_t b0 = 0; b0 < a.nb; b0 += kGetRowsBlocks) {
        const int nblk = (int) min<int64_t>(kGetRowsBlocks, a.nb - b0);
        const GrPass p{slice, (uint64_t) a.M * (uint64_t) a.nb, (uint64_t) g0 * a.nb, (uint64_t) rs, (uint64_t) lane, b0, nblk};
        // every load of the pass issued before the first is scattered into LDS: one memory round
        // trip per pass, not one per area
        GrArea<DT, 0> a0;
        GrArea<DT, 1> a1;
        GrArea<DT, 2> a2;
        a0.load(p);
        a1.load(p);
        a2.load(p);
        a0.scatter(p, nat, BB);
        a1.scatter(p, nat, BB);
        a2.scatter(p, nat, BB);
        __syncthreads();
        for (int e = threadIdx.x; e < nblk * BS; e += blockDim.x) y[b0 * BS + e] = deq_elem<DT>(nat + (e / BS) * BB, e % BS);
        __syncthreads();
    }
}

// GET_ROWS on F32 / F16 rows (natural layout, rows w_s1 bytes apart): one work-group per output
// row, each element widened exactly to f32 (the reference's load_float)
template <int DT>
__global__ __launch_bounds__(256) void k_get_rows_float(GetRowsArgs a, uint64_t w_s1) {
    const int64_t row = blockIdx.x;
    const int64_t c = row / (a.n0 * a.n1), rem = row - c * a.n0 * a.n1, bi = rem / a.n0, ai = rem - bi * a.n0;
    int64_t r = a.ids[ai * a.i_s0 + bi * a.i_s1 + c * a.i_s2];
    r = r < 0 ? 0 : (r >= a.M ? a.M - 1 : r); // out-of-range rows read the nearest row
    const uint8_t * src = a.w + (uint64_t) bi * a.w_s2 + (uint64_t) c * a.w_s3 + (uint64_t) r * w_s1;
    float * y = a.y + ai * a.y_s1 + bi * a.y_s2 + c * a.y_s3;
    for (int64_t e = threadIdx.x; e < a.K; e += blockDim.x) {
        if constexpr (DT == F32) y[e] = reinterpret_cast<const float *>(src)[e];
        else y[e] = __half2float(__ushort_as_half(reinterpret_cast<const unsigned short *>(src)[e]));
    }
}

unsigned grid_for(int64_t n, int threads) {
    const int64_t g = (n + threads - 1) / threads;
    return (unsigned) (g < 65536 * 8 ? (g < 1 ? 1 : g) : 65536 * 8);
}

} // namespace

hipError_t launch_r32_move(int dtype, int64_t K, int64_t M, int64_t row0, int64_t nrows, uint8_t * nat, uint8_t * rep, bool pack,
                           hipStream_t stream) {
    const Areas ar = areas_of(dtype);
    if (ar.na == 0 || nrows <= 0) return hipErrorInvalidValue;
    const int64_t nb = K / block_elems(dtype);
    const int64_t groups = (nrows + 31) / 32;
    if (groups > 65535) return hipErrorInvalidValue; // the caller chunks
    uint64_t before = 0;
    for (int k = 0; k < ar.na; ++k) {
        MoveArgs a;
        a.nat = nat;
        a.area = rep + (uint64_t) M * nb * before;
        a.M = M;
        a.nb = nb;
        a.row0 = row0;
        a.nrows = nrows;
        a.bs = block_bytes(dtype);
        a.src = ar.src[k];
        a.len = ar.len[k];
        a.xr = ar.xr[k];
        a.pack = pack ? 1 : 0;
        const int U = a.len == 2 ? 1 : a.len / 16;
        const int64_t per_group = 32 * nb * U;
        const unsigned gx = (unsigned) std::min<int64_t>((per_group + 255) / 256, 4096);
        hipLaunchKernelGGL(k_r32_move, dim3(gx, (unsigned) groups), dim3(256), 0, stream, a);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        before += (uint64_t) ar.len[k];
    }
    return hipSuccess;
}

hipError_t launch_get_rows(const GetRowsLaunch & g, hipStream_t stream) {
    const int64_t rows = g.n0 * g.n1 * g.n2;
    if (rows <= 0) return hipSuccess;
    if (rows > 0x7FFFFFFF) return hipErrorInvalidValue;
    GetRowsArgs a;
    a.w = g.w;
    a.w_s2 = g.w_s2;
    a.w_s3 = g.w_s3;
    a.ids = g.ids;
    a.i_s0 = g.i_s0;
    a.i_s1 = g.i_s1;
    a.i_s2 = g.i_s2;
    a.y = g.y;
    a.y_s1 = g.y_s1;
    a.y_s2 = g.y_s2;
    a.y_s3 = g.y_s3;
    a.K = g.K;
    a.M = g.M;
    a.n0 = g.n0;
    a.n1 = g.n1;
    const dim3 grid((unsigned) rows), block(256);
    if (g.dtype == F32 || g.dtype == F16) {
        a.nb = 0;
        if (g.dtype == F32) hipLaunchKernelGGL(k_get_rows_float<F32>, grid, block, 0, stream, a, g.w_s1);
        else hipLaunchKernelGGL(k_get_rows_float<F16>, grid, block, 0, stream, a, g.w_s1);
        return hipGetLastError();
    }
    a.nb = g.K / block_elems(g.dtype);
    static const bool areas_ok = gr_areas_match<Q4_0>() && gr_areas_match<Q8_0>() && gr_areas_match<Q4_K>() && gr_areas_match<Q6_K>();
    if (!areas_ok) return hipErrorInvalidValue;
    switch (g.dtype) {
        case Q4_0: hipLaunchKernelGGL(k_get_rows<Q4_0>, grid, block, 0, stream, a); break;
        case Q8_0: hipLaunchKernelGGL(k_get_rows<Q8_0>, grid, block, 0, stream, a); break;
        case Q4_K: hipLaunchKernelGGL(k_get_rows<Q4_K>, grid, block, 0, stream, a); break;
        case Q6_K: hipLaunchKernelGGL(k_get_rows<Q6_K>, grid, block, 0, stream, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dequantize(int dtype, const uint8_t * src, float * dst, int64_t n_blocks, hipStream_t stream) {
    const int64_t n = n_blocks * block_elems(dtype);
    const unsigned g = grid_for(n, 256);
    switch (dtype) {
        case Q4_0: hipLaunchKernelGGL(k_dequant<Q4_0>, dim3(g), dim3(256), 0, stream, src, dst, n); break;
        case Q8_0: hipLaunchKernelGGL(k_dequant<Q8_0>, dim3(g), dim3(256), 0, stream, src, dst, n); break;
        case Q4_K: hipLaunchKernelGGL(k_dequant<Q4_K>, dim3(g), dim3(256), 0, stream, src, dst, n); break;
        case Q6_K: hipLaunchKernelGGL(k_dequant<Q6_K>, dim3(g), dim3(256), 0, stream, src, dst, n); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_quantize(int dtype, const float * src, uint8_t * dst, int64_t n_blocks, hipStream_t stream) {
    const unsigned g = (unsigned) ((n_blocks + 127) / 128);
    if (n_blocks <= 0 || (n_blocks + 127) / 128 > 0x7FFFFFFF) return hipErrorInvalidValue;
    switch (dtype) {
        case Q4_0: hipLaunchKernelGGL(k_quant<Q4_0>, dim3(g), dim3(128), 0, stream, src, dst, n_blocks); break;
        case Q8_0: hipLaunchKernelGGL(k_quant<Q8_0>, dim3(g), dim3(128), 0, stream, src, dst, n_blocks); break;
        case Q4_K: hipLaunchKernelGGL(k_quant<Q4_K>, dim3(g), dim3(128), 0, stream, src, dst, n_blocks); break;
        case Q6_K: hipLaunchKernelGGL(k_quant<Q6_K>, dim3(g), dim3(128), 0, stream, src, dst, n_blocks); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_fill_normal(float * dst, int64_t n, uint64_t seed, float mean, float stddev, hipStream_t stream) {
    hipLaunchKernelGGL(k_fill_normal, dim3(grid_for(n, 256)), dim3(256), 0, stream, dst, n, seed, mean, stddev);
    return hipGetLastError();
}

} // namespace sgk
