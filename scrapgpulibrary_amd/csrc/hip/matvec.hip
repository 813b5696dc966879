// Decode matvec over R32 weights for 1 <= N <= 8 columns (gfx950, wave64).
//
// Replaces, for the hip backend, the reference's R32 matvec kernels k_mvr_* / k_mvrc_*
// (src/backends/opencl11/kernels/mul_mv_r.cl:240-287), k_mvr_q4_k / k_mvr_q6_k (mul_mv_k.cl:396-450)
// and, for 2-3 weights sharing x, k_mvm_* (mul_mv_multi.cl:46-99). Same products, new design.
//
// Work decomposition. A work-group owns a tile of 16 * RG rows (inside one R32 group of 32 rows)
// and all of K. Its W waves split K into contiguous ranges of steps (a step = 256 elements), so a
// wave only needs its own part of x, which it converts into its private LDS region; the waves
// meet once per tile, at the end, to add their partial row sums in a fixed order.
//
// Inside a wave, lane l serves row r = l % 16 (of each 16-row group) through part p = l / 16. A
// step's bytes of one row are dealt to the 4 parts by whole scale groups, so one 128-bit wave load
// reads four runs of 256 contiguous bytes of one R32 unit area.
//
// Integer dot products on the matrix cores. x is converted to int8 (below); the weights' integer
// codes (nibbles, 6-bit values, bytes) are unpacked to int8 in registers. One
// v_mfma_i32_16x16x64_i8 then takes the 16 rows' codes as its B operand (lane (r, p) supplies 16
// codes of row r: column r, k-group p) and x as its A operand. A decode product has only one x
// column, so the 16 rows of A are used to keep apart what must be scaled separately: rows 4w ..
// 4w + 2 of A (a "window") hold the three planes of x over one scale group, for the lanes whose
// k-group lies in that group, and zeros elsewhere (row 4w + 3 is zero). Lane (r, p) receives rows
// 4p .. 4p + 3 of D, so window p of each accumulator set is what lane part p scales: each format
// maps its MFMAs to accumulator sets so that every (set, window) holds exactly one scale group.
// Per 64 weights a lane spends ~30 VALU operations (unpack + scales) instead of ~110 with VALU dot
// products, which leaves the VALU idle enough to overlap the HBM stream.
//
// x conversion. Every 32-element segment of x is stored as three int8 planes a, b, c and a unit f
// (f = max|x| / (127 * 253)): x = f * (253 * a + b + c / 253) + e, plus the plain sums of its two
// 16-element halves:
//   sum_i q_i x_i ~= f * ((253 * sum q a + sum q b) + (sum q c) / 253)
// with each format's constant offset applied once per scale group through the segment sums:
//   Q4_0: d * (sum q x - 8 sum x)            Q8_0: d * sum q x      (q = stored byte xor 0x80)
//   Q4_K: d*sc * sum q x - dmin*m * sum x    Q6_K: d*sc * (sum q x - 32 sum x)
// |e| <= f / 506 = max|x_seg| / 16 257 146 (1.03 * 2^-24 of the segment's largest element), so each
// product carries x at the precision of an fp32 element of that magnitude. A segment with an Inf
// or NaN, or whose largest |x| is below 2^-90, is not converted: its planes and sums are zero and
// its products are formed in plain fp32 from the dequantized weights (seg_exact), so non-finite
// inputs give the reference's +-Inf / NaN pattern.
//
// Two forms:
//  * burst (N = 1, K <= 64 steps): one tile per work-group, at most 4 steps per wave; the wave
//    loads its x range, then issues every weight load, and only then converts x, so the x round
//    trip hides under the weight round trip. No loop-carried state: few registers, many waves per
//    SIMD, and the hardware dispatcher streams the work-groups.
//  * streaming (N > 1, or longer K): a persistent grid; each work-group walks tiles, its waves
//    convert their x range once (when it fits the LDS budget) and keep the next step's loads in
//    flight while computing the current one.
#include "kernels.h"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

namespace sgk {

LaunchForm & last_form() {
    thread_local LaunchForm f{{0}, 0};
    return f;
}
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kStep = 256;       // K elements per step
constexpr int kSegs = 8;         // 32-element x segments per step
constexpr int kLdsX = 64 * 1024; // bytes of converted x per work-group (all waves)

struct MvArgs {
    const uint8_t * w[3];
    int64_t M[3];
    float * y[3];
    int64_t ys1[3];
    int64_t tstart[4]; // matrix j owns tiles [tstart[j], tstart[j + 1])
    int64_t K, nb, nst; // elements, blocks and steps per row
    const float * x;
    int64_t x_s1, x_s2, x_s3;
    uint64_t w_s2, w_s3;
    int64_t y_s2, y_s3;
    int64_t ne12, r2, r3;
    int64_t tiles; // row tiles over all matrices
    int cs;        // steps per x chunk of one wave
    int xvec;      // x columns are 16-byte aligned: float4 loads
    // MUL_MAT_ID (ids != nullptr): blockIdx.y is the pair t * n_used + i
    const int32_t * ids;
    int64_t ids_s0, ids_s1, n_used, n_exp;
    int x_shared;
    // chunked burst (k_mvb with CHUNK): blockIdx.y is the K chunk (kChunkSteps steps each); part:
    // [chunk][tile * 16 RG + row] partial sums; arrive: chunks done per row tile, zero between
    // launches (the last chunk of a tile resets its count)
    int64_t nck;
    float * part;
    uint32_t * arrive;
};

constexpr int kChunkSteps = 16; // steps of K per work-group of the chunked burst (8 waves x 2)

__device__ __forceinline__ float half_bits(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short) (h & 0xFFFFu)));
}

// weight loads are non-temporal: every weight byte is read once per product, so it should not
// displace what the caches hold for the next launches (x, y, the counts). Measured on the Qwen3-8B
// decode token: 1.237 -> 1.153 ms (3.54 -> 3.79 TB/s; gate+up 12.9 -> 11.4 us, q+k+v 6.1 -> 5.3)
typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load16(const uint8_t * p) {
    const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t load_half(const uint8_t * p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
}

__device__ __forceinline__ v4i as_v4i(uint4 q) {
    v4i v;
    v.x = (int) q.x;
    v.y = (int) q.y;
    v.z = (int) q.z;
    v.w = (int) q.w;
    return v;
}

__device__ __forceinline__ v4i lo4(uint4 q) {
    return as_v4i(make_uint4(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu));
}
__device__ __forceinline__ v4i hi4(uint4 q) {
    return as_v4i(make_uint4((q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu, (q.z >> 4) & 0x0F0F0F0Fu, (q.w >> 4) & 0x0F0F0F0Fu));
}

__device__ __forceinline__ v4i mfma(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// (253 * A + B) + C / 253 over the three planes' integer sums, as float: 253 A + B is exact in
// float for every format (|A| <= 127 * 128 * 32), C enters with one rounding
__device__ __forceinline__ float planes(int da, int db, int dc) {
    return fmaf((float) dc, 1.0f / 253.0f, (float) (__mul24(da, 253) + db)); // (|A| < 2^23: one v_mad_i32_i24)
}
__device__ __forceinline__ float planes(const v4i & D) {
    return planes(D.x, D.y, D.z);
}

// one x segment in LDS: planes a, b, c (32 int8 each; plane k at byte 32 k, half h at + 16 h)
struct XSeg {
    uint4 a0, a1, b0, b1, c0, c1;
};
constexpr int kSegBytes = (int) sizeof(XSeg);

// The converted x of one wave's chunk, per column n: xs[n * nseg + g] (planes) and
// xf[n * nseg + g] = {f, sum of elements 0..15, sum of elements 16..31, sum of all 32}; f = -0.0
// flags a segment left to seg_exact.
// zpad: 16 zero bytes, the A operand of lanes that carry no x.
struct XView {
    const XSeg * xs;
    const float4 * xf;
    const uint8_t * zpad;
    int nseg;
};

__device__ __forceinline__ bool seg_flagged(const float4 & f) {
    return __float_as_uint(f.x) == 0x80000000u;
}

// ---- per format ----------------------------------------------------------------------------------
// init() resolves the lane's row in every R32 area once (Q4_K, Q8_0, Q4_0: as 32-bit byte offsets
// from the matrix slice's base w, which is uniform across the work-group and so stays in scalar
// registers; a slice is < 4 GiB, checked on the host); load(step) fetches what the lane needs of
// one step, branch-free; bop(raw, t) is the lane's B operand (16 int8 codes) for MFMA t = 0..3 of the step;
// aoff(t, c, k, g) is the byte offset, inside the step's XSeg run, of the 16 x bytes that lane
// (row 4c + k of A: window c, plane k; k-group g) supplies to MFMA t, or -1 for zeros; set(t) is
// the accumulator set MFMA t adds into; flush() scales the integer sums of lane part p (window p of
// each set) into the row sum.

template <int DT> struct Fmt;

// Q4_K: a step is one block; part p takes chunk p (64 elements: units 2p, 2p + 1 of the 128
// nibble bytes): sub-block 2p (low nibbles), 2p + 1 (high). MFMA t takes elements 64p + 16t .. +15
// (t = 0, 1: low nibbles of units 2p, 2p + 1; t = 2, 3: high nibbles). Set t / 2, window c:
// sub-block 2c + t / 2.
template <>
struct Fmt<Q4_K> {
    static constexpr int ND = 2; // accumulator sets per step
    __device__ static constexpr int set(int t) {
        return t >> 1;
    }
    struct Raw {
        uint4 q0, q1, hd;
    };
    const uint8_t * w;
    uint32_t qo, ho, u; // unit stride u = 16 * rows in the group; a block is 8 units
    int p;
    __device__ void init(const uint8_t * w_, int64_t M, int64_t nb, int64_t g0, int rs, int lr, int part) {
        w = w_;
        p = part;
        u = (uint32_t) rs * 16;
        qo = (uint32_t) (g0 * nb * 128 + lr * 16) + (uint32_t) (2 * p) * u;
        ho = (uint32_t) (M * nb * 128 + g0 * nb * 16 + lr * 16);
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        const uint32_t q = __umul24((uint32_t) step * 8, u) + qo;
        r.q0 = load16(w + q);
        r.q1 = load16(w + q + u);
        r.hd = load16(w + (__umul24((uint32_t) step, u) + ho));
        return r;
    }
    __device__ static v4i bop(const Raw & r, int t) {
        return t == 0 ? lo4(r.q0) : t == 1 ? lo4(r.q1) : t == 2 ? hi4(r.q0) : hi4(r.q1);
    }
    __device__ static int aoff(int t, int c, int k, int g) {
        if (c != g || k == 3) return -1;
        return (2 * g + (t >> 1)) * kSegBytes + k * 32 + (t & 1) * 16;
    }
    __device__ float flush(const Raw & r, const v4i * D, const float4 * xf) const {
        const float d = half_bits(r.hd.x), dmin = half_bits(r.hd.x >> 16);
        const uint32_t s0 = r.hd.y, s1 = r.hd.z, s2 = r.hd.w; // scale bytes 0..3, 4..7, 8..11
        // 6-bit scale and min of sub-blocks 2p, 2p + 1 (get_scale_min_k4)
        const int sh0 = 16 * (p & 1), sh1 = sh0 + 8;
        float sc0, m0, sc1, m1;
        if (p < 2) {
            sc0 = (float) ((s0 >> sh0) & 63u);
            m0 = (float) ((s1 >> sh0) & 63u);
            sc1 = (float) ((s0 >> sh1) & 63u);
            m1 = (float) ((s1 >> sh1) & 63u);
        } else {
            const uint32_t t0 = s2 >> sh0, t1 = s2 >> sh1;
            sc0 = (float) ((t0 & 0x0Fu) | (((s0 >> sh0) >> 2) & 0x30u));
            m0 = (float) (((t0 >> 4) & 0x0Fu) | (((s1 >> sh0) >> 2) & 0x30u));
            sc1 = (float) ((t1 & 0x0Fu) | (((s0 >> sh1) >> 2) & 0x30u));
            m1 = (float) (((t1 >> 4) & 0x0Fu) | (((s1 >> sh1) >> 2) & 0x30u));
        }
        const float4 f0 = xf[2 * p], f1 = xf[2 * p + 1];
        float a = (d * sc0) * f0.x * planes(D[0]);
        a = fmaf(-dmin * m0, f0.w, a);
        a = fmaf((d * sc1) * f1.x, planes(D[1]), a);
        return fmaf(-dmin * m1, f1.w, a);
    }
};

// Q6_K: a step is one block; part p takes task p = (h, hf): the 64 elements 128h + 32t + 16hf + i
// (t, i < 4, 16) built from ql units 4h + hf, 4h + 2 + hf and qh unit 8 + 2h + hf; MFMA t takes
// the 16 of run t, which has its own signed 8-bit scale. One accumulator set per MFMA; window c
// of set t: run t of task c.
template <>
struct Fmt<Q6_K> {
    static constexpr int ND = 4;
    __device__ static constexpr int set(int t) {
        return t;
    }
    struct Raw {
        uint4 qa, qc, qh, sc;
        uint32_t d;
    };
    const uint8_t * qb;
    const uint8_t * sb;
    const uint8_t * db;
    uint32_t qblk, qunit, sblk, dblk;
    int p;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb, int64_t g0, int rs, int lr, int part) {
        p = part;
        qb = w + (uint64_t) g0 * nb * 192 + (uint64_t) lr * 16;
        sb = w + (uint64_t) M * nb * 192 + (uint64_t) g0 * nb * 16 + (uint64_t) lr * 16;
        db = w + (uint64_t) M * nb * 208 + (uint64_t) g0 * nb * 2 + (uint64_t) lr * 2;
        qblk = (uint32_t) rs * 192;
        qunit = (uint32_t) rs * 16;
        sblk = (uint32_t) rs * 16;
        dblk = (uint32_t) rs * 2;
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        const int h = p >> 1, hf = p & 1;
        const uint8_t * b = qb + (uint32_t) step * qblk;
        r.qa = load16(b + (uint32_t) (4 * h + hf) * qunit);     // ql[64h + 16hf + i]
        r.qc = load16(b + (uint32_t) (4 * h + 2 + hf) * qunit); // ql[64h + 32 + 16hf + i]
        r.qh = load16(b + (uint32_t) (8 + 2 * h + hf) * qunit); // qh[32h + 16hf + i]
        r.sc = load16(sb + (uint32_t) step * sblk);
        r.d = load_half(db + (uint32_t) step * dblk);
        return r;
    }
    // 6-bit codes of run t: low nibbles of qa (t 0) / qc (t 1), high nibbles (t 2, 3), with bits
    // 2t, 2t + 1 of qh on top
    __device__ static v4i bop(const Raw & r, int t) {
        const uint4 ql = (t & 1) ? r.qc : r.qa;
        const int ls = t < 2 ? 0 : 4;
        const int hs = 2 * t;
        return as_v4i(make_uint4(((ql.x >> ls) & 0x0F0F0F0Fu) | (((r.qh.x >> hs) << 4) & 0x30303030u),
                                 ((ql.y >> ls) & 0x0F0F0F0Fu) | (((r.qh.y >> hs) << 4) & 0x30303030u),
                                 ((ql.z >> ls) & 0x0F0F0F0Fu) | (((r.qh.z >> hs) << 4) & 0x30303030u),
                                 ((ql.w >> ls) & 0x0F0F0F0Fu) | (((r.qh.w >> hs) << 4) & 0x30303030u)));
    }
    __device__ static int aoff(int t, int c, int k, int g) {
        if (c != g || k == 3) return -1;
        const int h = g >> 1, hf = g & 1;
        return (4 * h + t) * kSegBytes + k * 32 + hf * 16;
    }
    __device__ float flush(const Raw & r, const v4i * D, const float4 * xf) const {
        const int h = p >> 1, hf = p & 1;
        const float d = half_bits(r.d);
        // scale of run t: byte 8h + hf + 2t of the 16 (stored xor 0x80, so value = byte - 128)
        const uint32_t sw0 = h ? r.sc.z : r.sc.x, sw1 = h ? r.sc.w : r.sc.y;
        float a = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t sw = t < 2 ? sw0 : sw1;
            const float ds = d * ((float) ((sw >> (8 * (2 * (t & 1) + hf))) & 0xFFu) - 128.0f);
            const float4 f = xf[4 * h + t];
            const float s16 = hf ? f.z : f.y;
            a = fmaf(ds, fmaf(f.x, planes(D[t]), -32.0f * s16), a);
        }
        return a;
    }
};

// Q8_0: a step is 8 blocks of 32; MFMA t takes blocks 2t, 2t + 1 (part g: half g % 2 of block
// 2t + g / 2). Set t / 2, window 2 (t % 2) + g / 2 holds block 2t + g / 2, so part p scales blocks
// p (set 0) and p + 4 (set 1). Blocks past the end of the row (K % 256 != 0) load block 0 and
// contribute with d = 0.
template <>
struct Fmt<Q8_0> {
    static constexpr int ND = 2;
    __device__ static constexpr int set(int t) {
        return t >> 1;
    }
    struct Raw {
        uint4 u[4];
        uint32_t d0, d1;
    };
    const uint8_t * w;
    uint32_t qo, dof, u, nb; // block b: units 2b, 2b + 1 (2b u), d at b u / 8 in the d area
    int p;
    __device__ void init(const uint8_t * w_, int64_t M, int64_t nb_, int64_t g0, int rs, int lr, int part) {
        w = w_;
        p = part;
        nb = (uint32_t) nb_;
        u = (uint32_t) rs * 16;
        qo = (uint32_t) (g0 * nb_ * 32 + lr * 16) + (uint32_t) (p & 1) * u;
        dof = (uint32_t) (M * nb_ * 32 + g0 * nb_ * 2 + lr * 2);
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t b = (uint32_t) step * 8 + 2 * t + (p >> 1);
            b = b < nb ? b : 0;
            r.u[t] = load16(w + (__umul24(2 * b, u) + qo));
        }
        const uint32_t b0 = (uint32_t) step * 8 + p, b1 = b0 + 4;
        const uint32_t d0 = load_half(w + (__umul24(b0 < nb ? b0 : 0, u >> 3) + dof));
        const uint32_t d1 = load_half(w + (__umul24(b1 < nb ? b1 : 0, u >> 3) + dof));
        r.d0 = b0 < nb ? d0 : 0u;
        r.d1 = b1 < nb ? d1 : 0u;
        return r;
    }
    __device__ static v4i bop(const Raw & r, int t) {
        const uint4 q = r.u[t];
        return as_v4i(make_uint4(q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u));
    }
    __device__ static int aoff(int t, int c, int k, int g) {
        if (c != 2 * (t & 1) + (g >> 1) || k == 3) return -1;
        return (2 * t + (g >> 1)) * kSegBytes + k * 32 + (g & 1) * 16;
    }
    __device__ float flush(const Raw & r, const v4i * D, const float4 * xf) const {
        const float a = half_bits(r.d0) * xf[p].x * planes(D[0]);
        return fmaf(half_bits(r.d1) * xf[p + 4].x, planes(D[1]), a);
    }
};

// Q4_0: a step is 8 blocks of 32 (16 nibble bytes each: low nibbles = elements 0..15, high =
// 16..31); part p takes blocks p and p + 4. MFMA t: blocks 0..3 (t < 2) or 4..7, half t % 2.
// Set t / 2, window c: block c + 4 (t / 2).
template <>
struct Fmt<Q4_0> {
    static constexpr int ND = 2;
    __device__ static constexpr int set(int t) {
        return t >> 1;
    }
    struct Raw {
        uint4 qa, qb;
        uint32_t da, db;
    };
    const uint8_t * w;
    uint32_t qo, dof, u, nb; // block b: unit at b u, d at b u / 8 in the d area
    int p;
    __device__ void init(const uint8_t * w_, int64_t M, int64_t nb_, int64_t g0, int rs, int lr, int part) {
        w = w_;
        p = part;
        nb = (uint32_t) nb_;
        u = (uint32_t) rs * 16;
        qo = (uint32_t) (g0 * nb_ * 16 + lr * 16);
        dof = (uint32_t) (M * nb_ * 16 + g0 * nb_ * 2 + lr * 2);
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        uint32_t ba = (uint32_t) step * 8 + p, bb = ba + 4;
        const bool oka = ba < nb, okb = bb < nb;
        ba = oka ? ba : 0;
        bb = okb ? bb : 0;
        r.qa = load16(w + (__umul24(ba, u) + qo));
        r.qb = load16(w + (__umul24(bb, u) + qo));
        const uint32_t da = load_half(w + (__umul24(ba, u >> 3) + dof));
        const uint32_t db = load_half(w + (__umul24(bb, u >> 3) + dof));
        r.da = oka ? da : 0u;
        r.db = okb ? db : 0u;
        return r;
    }
    __device__ static v4i bop(const Raw & r, int t) {
        return t == 0 ? lo4(r.qa) : t == 1 ? hi4(r.qa) : t == 2 ? lo4(r.qb) : hi4(r.qb);
    }
    __device__ static int aoff(int t, int c, int k, int g) {
        if (c != g || k == 3) return -1;
        return (g + 4 * (t >> 1)) * kSegBytes + k * 32 + (t & 1) * 16;
    }
    __device__ float flush(const Raw & r, const v4i * D, const float4 * xf) const {
        const float4 fa = xf[p], fb = xf[p + 4];
        const float a = half_bits(r.da) * fmaf(fa.x, planes(D[0]), -8.0f * fa.w);
        return fmaf(half_bits(r.db), fmaf(fb.x, planes(D[1]), -8.0f * fb.w), a);
    }
};

// The lane's A operand addressing: byte offsets inside a step's XSeg run for MFMAs t = 0..3, or
// -1 (zeros). Row of A = l % 16 = 4c + k, k-group g = l / 16.
template <int DT>
struct ALane {
    int off[4];
    __device__ explicit ALane(int lane) {
        const int row = lane & 15, c = row >> 2, k = row & 3, g = lane >> 4;
#pragma unroll
        for (int t = 0; t < 4; ++t) off[t] = Fmt<DT>::aoff(t, c, k, g);
    }
};

// One step of RG row groups (raw[i] = rows r + 16 i) for NC columns: accumulates into acc[i][n].
// sg0 = index of the step's first segment in the chunk.
template <int DT, int RG, int NC>
__device__ __forceinline__ void step_mfma(const Fmt<DT> (&f)[RG], const typename Fmt<DT>::Raw (&raw)[RG], const ALane<DT> & al, int sg0,
                                          const XView & xv, float (&acc)[RG][NC]) {
    constexpr int ND = Fmt<DT>::ND;
#pragma unroll
    for (int n = 0; n < NC; ++n) {
        const uint8_t * base = reinterpret_cast<const uint8_t *>(xv.xs + n * xv.nseg + sg0);
        v4i Aop[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint8_t * pa = al.off[t] >= 0 ? base + al.off[t] : xv.zpad;
            Aop[t] = *reinterpret_cast<const v4i *>(pa);
        }
        const float4 * xf = xv.xf + n * xv.nseg + sg0;
#pragma unroll
        for (int i = 0; i < RG; ++i) {
            v4i D[ND];
#pragma unroll
            for (int u = 0; u < ND; ++u) D[u] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int u = Fmt<DT>::set(t);
                D[u] = mfma(Aop[t], Fmt<DT>::bop(raw[i], t), D[u]);
            }
            acc[i][n] += f[i].flush(raw[i], D, xf);
        }
    }
}

// ---- x conversion ----------------------------------------------------------------------------------

// Segment g (of nseg) of a wave's range, elements 8q .. 8q + 7 held by this lane in v (lanes
// 4k .. 4k + 3 hold one segment): three int8 planes, the unit f and the plain sums. Rounding to
// integers: adding 1.5 * 2^23 leaves the nearest integer in the low mantissa bits. Each residual is
// one fma over an exact product (253 a and b are integers below 2^24), so x - f (253 a + b + c / 253)
// is only the last plane's rounding. Returns true for a segment flagged for seg_exact (non-finite,
// or largest |x| below 2^-90), whose planes and sums are zero and whose f is -0.0.
// (SPLIT: the unit and the sum of all 32 go to fo[g] and so[g] instead of xf[g])
template <bool SPLIT = false>
__device__ __forceinline__ bool convert_seg(const float (&v)[8], int g, int nseg, int q, XSeg * xs, float4 * xf, float * fo = nullptr,
                                            float * so = nullptr) {
    constexpr float kMagic = 12582912.0f; // 1.5 * 2^23
    float amax = 0.0f;
    int nonfinite = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float a = fabsf(v[i]);
        nonfinite |= !(a <= 3.40282347e38f); // Inf or NaN
        amax = fmaxf(amax, a);
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    nonfinite |= __shfl_xor(nonfinite, 1);
    nonfinite |= __shfl_xor(nonfinite, 2);
    const bool special = nonfinite || (amax > 0.0f && amax < 0x1p-90f);
    float t[8], sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        t[i] = special ? 0.0f : v[i];
        sum += t[i];
    }
    const float s16 = sum + __shfl_xor(sum, 1);
    const float s32 = s16 + __shfl_xor(s16, 2);
    const float s16o = __shfl_xor(s16, 2);
    const float f = special ? 0.0f : amax * (1.0f / 32131.0f); // 127 * 253
    const bool live = f > 0.0f && !special;
    // reciprocals need not be exact: |a| <= 127 holds within a few ulps, and a rounding off by one
    // near a tie leaves |b| <= 126.5 + tiny, |c| likewise
    const float ia = live ? __builtin_amdgcn_rcpf(253.0f * f) : 0.0f;
    const float ib = live ? __builtin_amdgcn_rcpf(f) : 0.0f;
    const float ic = 253.0f * ib;
    uint32_t pk[3][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint32_t ba[4], bb[4], bc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float x = t[4 * h + i];
            const float fa = fmaf(x, ia, kMagic);
            const float r1 = fmaf((kMagic - fa) * 253.0f, f, x); // x - 253 a f
            const float fb = fmaf(r1, ib, kMagic);
            const float r2 = fmaf(kMagic - fb, f, r1); // r1 - b f
            const float fc = fmaf(r2, ic, kMagic);
            ba[i] = __float_as_uint(fa);
            bb[i] = __float_as_uint(fb);
            bc[i] = __float_as_uint(fc);
        }
        // byte i of the result = byte 0 of word i
        pk[0][h] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(ba[3], ba[2], 0x0c0c0400u), __builtin_amdgcn_perm(ba[1], ba[0], 0x0c0c0400u),
                                         0x05040100u);
        pk[1][h] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(bb[3], bb[2], 0x0c0c0400u), __builtin_amdgcn_perm(bb[1], bb[0], 0x0c0c0400u),
                                         0x05040100u);
        pk[2][h] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(bc[3], bc[2], 0x0c0c0400u), __builtin_amdgcn_perm(bc[1], bc[0], 0x0c0c0400u),
                                         0x05040100u);
    }
    if (g < nseg) {
        uint8_t * sp = reinterpret_cast<uint8_t *>(xs + g);
#pragma unroll
        for (int k = 0; k < 3; ++k) *reinterpret_cast<uint2 *>(sp + 32 * k + 8 * q) = make_uint2(pk[k][0], pk[k][1]);
        if constexpr (SPLIT) {
            if (q == 0) {
                fo[g] = special ? -0.0f : f;
                so[g] = special ? 0.0f : s32;
            }
        } else {
            if (q == 0) xf[g] = special ? make_float4(-0.0f, 0.0f, 0.0f, 0.0f) : make_float4(f, s16, s16o, s32);
        }
    }
    return special && g < nseg;
}

// The wave's chunk of nseg segments starting at element e0, for NC columns. Lane l converts
// elements 8 (l % 4) .. +8 of segment l / 4 (16 segments per pass); elements past K are zero.
template <int NC>
__device__ bool convert_x(const MvArgs & A, const float * x, int64_t e0, int nseg, int lane, XSeg * xs, float4 * xf) {
    const int q = lane & 3;
    bool special = false;
    for (int base = 0; base < nseg; base += 16) {
        const int g = base + (lane >> 2);
        const int64_t e = e0 + 32 * (int64_t) g + 8 * q;
#pragma unroll 1
        for (int n = 0; n < NC; ++n) {
            float v[8];
            const float * xp = x + n * A.x_s1 + e;
            if (g < nseg && e < A.K) {
                if (A.xvec) {
                    const float4 u = *reinterpret_cast<const float4 *>(xp);
                    const float4 w = *reinterpret_cast<const float4 *>(xp + 4);
                    v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
                    v[4] = w.x; v[5] = w.y; v[6] = w.z; v[7] = w.w;
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[i] = xp[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = 0.0f;
            }
            special |= convert_seg(v, g, nseg, q, xs + n * nseg, xf + n * nseg);
        }
    }
    return __ballot(special) != 0; // wave-uniform: some segment needs seg_exact
}

// the slice a work-group works on
struct Where {
    int64_t y_off; // element offset of the slice's (pair's) output in y
    uint64_t w_off;
    const float * x;
};

// (32-bit divisions: slice counts are < 65536; the common single-slice case divides nothing, so
// the first loads issue right away)
__device__ __forceinline__ Where where_of(const MvArgs & A) {
    Where w;
    if (A.ids != nullptr) {
        // MUL_MAT_ID: the pair's expert, read once per work-group (a uniform scalar load)
        const uint32_t pr = blockIdx.y, nu = (uint32_t) A.n_used;
        const uint32_t t = pr / nu, i = pr - t * nu;
        int32_t e = A.ids[(int64_t) i * A.ids_s0 + (int64_t) t * A.ids_s1];
        e = e < 0 ? 0 : (e >= (int32_t) A.n_exp ? (int32_t) A.n_exp - 1 : e);
        w.w_off = (uint64_t) e * A.w_s2;
        w.x = A.x + (A.x_shared ? 0 : (int64_t) i * A.x_s1) + (int64_t) t * A.x_s2;
        w.y_off = (int64_t) i * A.ys1[0] + (int64_t) t * A.y_s2;
        return w;
    }
    if (gridDim.y == 1) {
        w.y_off = 0;
        w.w_off = 0;
        w.x = A.x;
        return w;
    }
    const uint32_t sl = blockIdx.y, ne12 = (uint32_t) A.ne12;
    const uint32_t i2 = sl % ne12, i3 = sl / ne12;
    w.y_off = (int64_t) i2 * A.y_s2 + (int64_t) i3 * A.y_s3;
    w.w_off = (uint64_t) (i2 / (uint32_t) A.r2) * A.w_s2 + (uint64_t) (i3 / (uint32_t) A.r3) * A.w_s3;
    w.x = A.x + (int64_t) i2 * A.x_s2 + (int64_t) i3 * A.x_s3;
    return w;
}

// where_of for the burst form's MUL_MAT_ID instances (ids present) in two halves, so that the
// pair's expert id is not a round trip ahead of its x loads: where_first() needs no memory read
// and issues the id load (a vector load from one address: its wait counts in order, so the x
// loads issued after it stay in flight), where_second() turns the id into the weight offset once
// the x loads are out.
__device__ __forceinline__ Where where_first(const MvArgs & A, int32_t & eid) {
    Where w;
    const uint32_t pr = blockIdx.y, nu = (uint32_t) A.n_used;
    const uint32_t t = pr / nu, i = pr - t * nu;
    eid = __hip_atomic_load(A.ids + (int64_t) i * A.ids_s0 + (int64_t) t * A.ids_s1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    w.w_off = 0;
    w.x = A.x + (A.x_shared ? 0 : (int64_t) i * A.x_s1) + (int64_t) t * A.x_s2;
    w.y_off = (int64_t) i * A.ys1[0] + (int64_t) t * A.y_s2;
    return w;
}
__device__ __forceinline__ void where_second(const MvArgs & A, int32_t eid, Where & w) {
    int32_t e = __builtin_amdgcn_readfirstlane(eid);
    e = e < 0 ? 0 : (e >= (int32_t) A.n_exp ? (int32_t) A.n_exp - 1 : e);
    w.w_off = (uint64_t) e * A.w_s2;
}

// the lane's rows of a tile of 16 * RG rows: f[i] serves row m0 + r + 16 i (dead lanes of a
// partial last tile read a real row and drop the result)
struct Row {
    int j;
    int64_t M, m0;
};

template <int DT, int RG>
__device__ __forceinline__ Row row_of(const MvArgs & A, int64_t tile, uint64_t w_off, int r, int part, Fmt<DT> (&f)[RG]) {
    constexpr int R = 16 * RG;
    const int j = tile >= A.tstart[1] ? (tile >= A.tstart[2] ? 2 : 1) : 0;
    const int64_t M = A.M[j];
    const int64_t m0 = (tile - A.tstart[j]) * R;
#pragma unroll
    for (int i = 0; i < RG; ++i) {
        // each 16-row group lies in one R32 group (48-row tiles straddle two); rows past M
        // read the last row (their results are not stored)
        const int64_t m = min(m0 + r + 16 * i, M - 1);
        const int64_t g0 = m & ~(int64_t) 31;
        f[i].init(A.w[j] + w_off, M, A.nb, g0, (int) min<int64_t>(32, M - g0), (int) (m - g0), part);
    }
    return Row{j, M, m0};
}

// Adds the parts of each row (lanes r, r + 16, r + 32, r + 48) and then the waves in order; lanes
// tid < 16 * RG * NC write y. red: [W][NC][16 * RG] floats.
// fix() runs after this wave's sums are in red (the exact sums of flagged x segments go there)
struct NoFix {
    __device__ void operator()() const {}
};
template <int RG, int NC, int W, class Fix = NoFix>
__device__ __forceinline__ void reduce_store(const MvArgs & A, const Where & wh, const Row & row, float (&acc)[RG][NC], float * red, int tid,
                                             const Fix & fix = Fix()) {
    constexpr int R = 16 * RG;
    const int lane = tid & 63, wave = tid >> 6, r = lane & 15;
#pragma unroll
    for (int i = 0; i < RG; ++i) {
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            float v = acc[i][n];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            if (lane < 16) red[(wave * NC + n) * R + 16 * i + r] = v;
        }
    }
    fix();
    __syncthreads();
    if (tid < NC * R) {
        const int n = tid / R, rr = tid % R;
        const int64_t m = row.m0 + rr;
        if (m < row.M) {
            float v = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < W; ++w2) v += red[(w2 * NC + n) * R + rr];
            A.y[row.j][wh.y_off + n * A.ys1[row.j] + m] = v;
        }
    }
}

// ---- exact fp32 products over flagged x segments ---------------------------------------------------
//
// A segment that convert_seg flags (an Inf or NaN in it, or its largest |x| below 2^-90) has zero
// planes and sums; its products are formed here in fp32 instead, w[m, k] * x[k] with the weight
// dequantized by the reference's element formulas (src/core/ref/quant.cpp:30-108), so that +-Inf,
// Inf * 0 = NaN and NaN reach y as in the reference's fp32 dot product (ops.cpp:968-980). Only
// waves whose x holds such a segment take this path (a wave-uniform branch).

// one row of an R32 slice
struct R32Row {
    const uint8_t * w; // the slice
    int64_t M, nb, g0;
    int rs, lane;
};

__device__ __forceinline__ R32Row r32_row(const uint8_t * w, int64_t M, int64_t nb, int64_t m) {
    m = min(m, M - 1);
    const int64_t g0 = m & ~(int64_t) 31;
    return R32Row{w, M, nb, g0, (int) min<int64_t>(32, M - g0), (int) (m - g0)};
}

// natural byte j of block b of the row: area k of the slice starts at M nb (bytes per block of
// the earlier areas); in an area of L bytes per block, 16-byte unit u of block b of the row sits at
// g0 nb L + ((b L / 16 + u) rs + lane) 16, and a 2-byte area holds halves at g0 nb 2 + (b rs + lane)
// 2; the area's xor mask is undone
template <int DT>
__device__ uint32_t nat_byte(const R32Row & r, int64_t b, int j) {
    int before, src, len;
    uint32_t xr = 0;
    if constexpr (DT == Q4_0) {
        if (j >= 2) { before = 0; src = 2; len = 16; } else { before = 16; src = 0; len = 2; }
    } else if constexpr (DT == Q8_0) {
        if (j >= 2) { before = 0; src = 2; len = 32; xr = 0x80; } else { before = 32; src = 0; len = 2; }
    } else if constexpr (DT == Q4_K) {
        if (j >= 16) { before = 0; src = 16; len = 128; } else { before = 128; src = 0; len = 16; }
    } else {
        if (j < 192) { before = 0; src = 0; len = 192; }
        else if (j < 208) { before = 192; src = 192; len = 16; xr = 0x80; }
        else { before = 208; src = 208; len = 2; }
    }
    const uint8_t * area = r.w + (uint64_t) r.M * (uint64_t) r.nb * (uint64_t) before;
    const int o = j - src;
    const uint8_t * q = len == 2 ? area + (uint64_t) r.g0 * r.nb * 2 + ((uint64_t) b * r.rs + r.lane) * 2 + o
                                 : area + (uint64_t) r.g0 * r.nb * len + (((uint64_t) b * (len / 16) + o / 16) * r.rs + r.lane) * 16 + o % 16;
    return (uint32_t) *q ^ xr;
}

// weight [m, k] (the reference's dequantize_row_* element formulas)
template <int DT>
__device__ float weight_at(const R32Row & r, int64_t k) {
    constexpr int BS = DT == Q4_K || DT == Q6_K ? 256 : 32;
    const int64_t b = k / BS;
    const int i = (int) (k - b * BS);
    auto byte = [&](int j) { return nat_byte<DT>(r, b, j); };
    auto half = [&](int j) { return half_bits(byte(j) | (byte(j + 1) << 8)); };
    if constexpr (DT == Q4_0) {
        const uint32_t q = byte(2 + (i & 15));
        return (float) ((int) (i < 16 ? (q & 15u) : (q >> 4)) - 8) * half(0);
    } else if constexpr (DT == Q8_0) {
        return (float) (int8_t) byte(2 + i) * half(0);
    } else if constexpr (DT == Q4_K) {
        const int c = i / 64, l = i % 32, hi = (i % 64) >= 32, j = 2 * c + hi;
        uint32_t sc, mn;
        if (j < 4) {
            sc = byte(4 + j) & 63u;
            mn = byte(8 + j) & 63u;
        } else {
            sc = (byte(8 + j) & 15u) | ((byte(j) >> 6) << 4);
            mn = (byte(8 + j) >> 4) | ((byte(4 + j) >> 6) << 4);
        }
        const float d1 = half(0) * (float) sc, m1 = half(2) * (float) mn;
        const uint32_t q = byte(16 + 32 * c + l);
        return d1 * (float) (hi ? (q >> 4) : (q & 15u)) - m1;
    } else {
        const int h = i / 128, rr = (i % 128) / 32, l = i % 32;
        const uint32_t qh = byte(128 + 32 * h + l);
        const uint32_t lowq = byte(64 * h + l + ((rr & 1) ? 32 : 0));
        const int nib = (int) (rr < 2 ? (lowq & 15u) : (lowq >> 4));
        const int v = (nib | (int) (((qh >> (2 * rr)) & 3u) << 4)) - 32;
        const int sc = (int) (int8_t) byte(192 + 8 * h + 2 * rr + l / 16);
        return half(208) * (float) sc * (float) v;
    }
}

// the fp32 dot product of one row with x over the 32-element segment at k0: lane part p takes
// elements k0 + p + 4 i, then the four parts' sums are added, so every lane of the row returns
// the segment's sum
template <int DT>
__device__ __noinline__ float seg_exact(R32Row r, const float * x, int64_t k0, int p) {
    float s = 0.0f;
#pragma unroll 1
    for (int i = 0; i < 8; ++i) {
        const int64_t k = k0 + p + 4 * i;
        s += weight_at<DT>(r, k) * x[k];
    }
    s += __shfl_xor(s, 16);
    s += __shfl_xor(s, 32);
    return s;
}

// the flag of segment g of a view, the same on every lane (scalar: the branches on it stay uniform)
__device__ __forceinline__ bool flagged_at(const float4 * xf, int g) {
    return __builtin_amdgcn_readfirstlane(__float_as_uint(xf[g].x)) == 0x80000000u;
}

// one column, the single-column lane mapping (k_mvb): red[16 i + r] (this wave's row sums, lanes
// r < 16) += the exact sums of the flagged segments 0 .. nseg - 1 of the view (segment g starts
// at element k0 + 32 g) for rows m0 + 16 i + r of the slice w. Runs after the MFMA sums are
// stored, so that no accumulator is live; not inlined, and given only uniform values, so that
// it costs the main path no registers.
template <int DT, int RG>
__device__ __noinline__ void exact_red(const uint8_t * w, int64_t M, int64_t nb, int64_t m0, const float * x, const float4 * xf, int nseg,
                                       int64_t k0, float * red) {
    const int lane = threadIdx.x & 63;
    for (int g = 0; g < nseg; ++g) {
        if (!flagged_at(xf, g)) continue;
#pragma unroll
        for (int i = 0; i < RG; ++i) {
            const float e = seg_exact<DT>(r32_row(w, M, nb, m0 + (lane & 15) + 16 * i), x, k0 + 32 * (int64_t) g, lane >> 4);
            if (lane < 16) red[16 * i + lane] += e;
        }
    }
}

// the same for one column of k_mvc (16 rows at m0), the flagged segments given as bit g * bs of
// fmask
template <int DT>
__device__ __noinline__ void exact_red_n(const uint8_t * w, int64_t M, int64_t nb, int64_t m0, const float * x, uint64_t fmask, int bs, int nseg,
                                         int64_t k0, float * red) {
    const int lane = threadIdx.x & 63;
    for (int g = 0; g < nseg; ++g) {
        if (!((fmask >> (g * bs)) & 1u)) continue;
        const float e = seg_exact<DT>(r32_row(w, M, nb, m0 + (lane & 15)), x, k0 + 32 * (int64_t) g, lane >> 4);
        if (lane < 16) red[lane] += e;
    }
}

// single-column lane mapping (k_mvs): acc[i][n] of lane part 0 += the exact sums of the
// flagged segments sg .. sg + cnt - 1 of the view (segment sg + g starts at element k0 + 32 g)
template <int DT, int RG, int NC>
__device__ void exact_segments(const MvArgs & A, const Where & wh, const Row & row, int r, int part, const XView & xv, int sg, int cnt,
                               int64_t k0, float (&acc)[RG][NC]) {
    const uint8_t * w = A.w[row.j] + wh.w_off;
    for (int n = 0; n < NC; ++n) {
        for (int g = 0; g < cnt; ++g) {
            if (!flagged_at(xv.xf + n * xv.nseg, sg + g)) continue;
#pragma unroll
            for (int i = 0; i < RG; ++i) {
                const float e = seg_exact<DT>(r32_row(w, row.M, A.nb, row.m0 + r + 16 * i), wh.x + n * A.x_s1, k0 + 32 * (int64_t) g, part);
                if (part == 0) acc[i][n] += e;
            }
        }
    }
}

// The sum over c = 0 .. n - 1 of p[c stride], added in order of c (the chunk hand-overs below):
// agent-scope loads (coherent across XCDs by themselves), issued in batches of 8 before any is
// added, so the last chunk pays one memory round trip per 8 chunks instead of one per chunk.
__device__ __forceinline__ float ordered_sum(const float * p, int64_t stride, int64_t n) {
    float t = 0.0f;
    for (int64_t c0 = 0; c0 < n; c0 += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = c0 + i < n ? __hip_atomic_load(p + (c0 + i) * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (c0 + i < n) t += v[i];
    }
    return t;
}

// Burst form (one column, <= SPW steps per wave, one tile of 16 * RG rows per work-group): the wave
// first loads its x range, then issues its first step's weight loads, converts x, and then issues
// the loads of its other steps.
// CHUNK (one slice, W x SPW = kChunkSteps): work-group (tile, c) takes chunk c of K,
// so that a long K runs on several small work-groups instead of one large one per tile. The
// chunks' partial sums meet as in k_mvc: agent-scope stores, an arrival count per tile, and the
// last chunk to arrive adds them in chunk order and resets the count.
template <int DT, int RG, int W, int SPW, bool CHUNK = false, bool ID = false>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(SPW <= 2 && RG == 1 ? 6 : SPW <= 2 && RG == 2 ? 5 : 4, 8))) void k_mvb(MvArgs A) {
    static_assert(!CHUNK || W * SPW == kChunkSteps, "chunks of kChunkSteps steps");
    static_assert(!(CHUNK && ID), "MUL_MAT_ID pairs take whole K");
    using F = Fmt<DT>;
    using Raw = typename F::Raw;
    extern __shared__ uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int32_t eid = 0;
    Where wh = CHUNK ? Where{0, 0, A.x} : ID ? where_first(A, eid) : where_of(A);

    // the work-group's steps: all of K, or chunk blockIdx.y (CHUNK)
    const int64_t cb = CHUNK ? (int64_t) blockIdx.y * kChunkSteps : 0;
    const int64_t cn = CHUNK ? min<int64_t>(kChunkSteps, A.nst - cb) : A.nst;
    const int64_t s0 = cb + cn * wave / W, s1 = cb + cn * (wave + 1) / W;
    const int ns = (int) (s1 - s0);

    // x: lane l holds elements 8 (l % 4) .. +8 of segment l / 4 + 16 p of the wave's range (pass p)
    constexpr int XP = (SPW * kSegs + 15) / 16;
    float xv[XP][8];
    const int nseg = ns * kSegs;
    // every load below is unconditional (out-of-range ones read a valid address and are
    // discarded by a select), so the wait before the x conversion counts only the x loads: the
    // conversion overlaps the weight loads instead of waiting for the last of them
#pragma unroll
    for (int p = 0; p < XP; ++p) {
        const int g = 16 * p + (lane >> 2);
        const int64_t e = s0 * kStep + 32 * (int64_t) g + 8 * (lane & 3);
        const bool ok = g < nseg && e < A.K;
        const float * xp = wh.x + (ok ? e : 0);
        const float4 u = *reinterpret_cast<const float4 *>(xp);
        const float4 w = *reinterpret_cast<const float4 *>(xp + 4);
        xv[p][0] = ok ? u.x : 0.0f; xv[p][1] = ok ? u.y : 0.0f; xv[p][2] = ok ? u.z : 0.0f; xv[p][3] = ok ? u.w : 0.0f;
        xv[p][4] = ok ? w.x : 0.0f; xv[p][5] = ok ? w.y : 0.0f; xv[p][6] = ok ? w.z : 0.0f; xv[p][7] = ok ? w.w : 0.0f;
    }

    // the x loads stay ahead of the weight loads
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (ID) where_second(A, eid, wh);
    F f[RG];
    const Row row = row_of<DT, RG>(A, blockIdx.x, wh.w_off, lane & 15, lane >> 4, f);
    Raw buf[SPW][RG];
    // step 0's loads go out before the x conversion, the others after it: a wave stalls issuing
    // loads once the memory pipeline is full, and x converted behind all of them was the last
    // thing a work-group waited for (the decode token 1.18 -> 1.12 ms on one box)
    constexpr int S0 = 1;
#pragma unroll
    for (int s = 0; s < S0; ++s) {
        const int64_t ss = s < ns ? s0 + s : s0; // steps past the wave's range: reloaded, unused
#pragma unroll
        for (int i = 0; i < RG; ++i) buf[s][i] = f[i].load(ss);
    }
    __builtin_amdgcn_sched_barrier(0);

    XSeg * xs = reinterpret_cast<XSeg *>(lds) + (size_t) wave * SPW * kSegs;
    float4 * xf = reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * SPW * kSegs) + (size_t) wave * SPW * kSegs;
    float * red = reinterpret_cast<float *>(reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * SPW * kSegs) +
                                            (size_t) W * SPW * kSegs);
    uint8_t * zpad = reinterpret_cast<uint8_t *>(red + W * 16 * RG);
    if (lane < 4) reinterpret_cast<uint32_t *>(zpad)[lane] = 0u;
    bool sp = false;
#pragma unroll
    for (int p = 0; p < XP; ++p) sp |= convert_seg(xv[p], 16 * p + (lane >> 2), nseg, lane & 3, xs, xf);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = S0; s < SPW; ++s) {
        const int64_t ss = s < ns ? s0 + s : s0;
#pragma unroll
        for (int i = 0; i < RG; ++i) buf[s][i] = f[i].load(ss);
    }
    __builtin_amdgcn_sched_barrier(0);
    const bool special = __ballot(sp) != 0;
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();

    const ALane<DT> al(lane);
    const XView xw{xs, xf, zpad, nseg};
    float acc[RG][1];
#pragma unroll
    for (int i = 0; i < RG; ++i) acc[i][0] = 0.0f;
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
        if (s < ns) step_mfma<DT, RG, 1>(f, buf[s], al, s * kSegs, xw, acc);
    }
    if constexpr (!CHUNK) {
        reduce_store<RG, 1, W>(A, wh, row, acc, red, tid, [&] {
            if (special) exact_red<DT, RG>(A.w[row.j] + wh.w_off, row.M, A.nb, row.m0, wh.x, xf, nseg, s0 * kStep, red + wave * 16 * RG);
        });
    } else {
        // the waves' sums of the chunk (as reduce_store), then the chunks' through memory
        constexpr int R = 16 * RG;
        const int r = lane & 15;
#pragma unroll
        for (int i = 0; i < RG; ++i) {
            float v = acc[i][0];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            if (lane < 16) red[wave * R + 16 * i + r] = v;
        }
        if (special) exact_red<DT, RG>(A.w[row.j] + wh.w_off, row.M, A.nb, row.m0, wh.x, xf, nseg, s0 * kStep, red + wave * R);
        __syncthreads();
        const int64_t tile = blockIdx.x;
        if (tid < R) {
            float t = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < W; ++w2) t += red[w2 * R + tid];
            // agent-scope stores (written through the XCD's L2), waited for by this wave
            __hip_atomic_store(A.part + ((int64_t) blockIdx.y * A.tiles + tile) * R + tid, t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0)
        }
        // the count moves after this wave's write-through stores are acknowledged (vmcnt(0)
        // above): every chunk's sums are in memory before its increment is visible (the ordering
        // a release would give, without its L2 write-back)
        uint32_t & last = *reinterpret_cast<uint32_t *>(zpad + 16);
        if (tid == 0) last = __hip_atomic_fetch_add(A.arrive + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t) A.nck - 1;
        __syncthreads();
        // the last chunk of the tile to arrive adds all of them in chunk order and leaves the
        // count at zero for the next launch. Its loads are agent-scope (coherent across XCDs by
        // themselves, never served from a stale line of this XCD's L2) and issue only after the
        // count's atomic returned (the barrier that publishes `last`)
        if (last && tid < R) {
            const int64_t m = row.m0 + tid;
            const float t = ordered_sum(A.part + tile * R + tid, A.tiles * R, A.nck);
            if (m < row.M) A.y[row.j][m] = t;
            if (tid == 0) __hip_atomic_store(A.arrive + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Streaming form: one work-group walks tiles blockIdx.x, blockIdx.x + gridDim.x, ... (16 rows
// each). Its waves keep the same K range for every tile, so each converts its x range once (when
// the range fits the LDS budget; otherwise per chunk of cs steps and tile). The next step's loads
// (of this tile or the first of the next) are in flight while the current step is computed.
template <int DT, int NC, int W>
__global__ __launch_bounds__(64 * W) void k_mvs(MvArgs A) {
    using F = Fmt<DT>;
    using Raw = typename F::Raw;
    extern __shared__ uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, part = lane >> 4;
    const Where wh = where_of(A);

    const int64_t s0 = A.nst * wave / W, s1 = A.nst * (wave + 1) / W;
    const int ns = (int) (s1 - s0);
    const int cs = A.cs;
    const bool once = cs >= ns; // the wave's whole x range stays in LDS for all tiles
    XSeg * xs = reinterpret_cast<XSeg *>(lds) + (size_t) wave * cs * kSegs * NC;
    float4 * xf = reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * cs * kSegs * NC) + (size_t) wave * cs * kSegs * NC;
    float * red = reinterpret_cast<float *>(reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * cs * kSegs * NC) +
                                            (size_t) W * cs * kSegs * NC); // [2][W][NC][16]
    uint8_t * zpad = reinterpret_cast<uint8_t *>(red + 2 * W * NC * 16);
    if (lane < 4) reinterpret_cast<uint32_t *>(zpad)[lane] = 0u;
    const ALane<DT> al(lane);

    int64_t tile = blockIdx.x;
    F f[1], fn[1];
    Row row = row_of<DT, 1>(A, tile, wh.w_off, r, part, f);
    Raw cur[1];
    if (ns > 0) cur[0] = f[0].load(s0);
    bool special = false; // the current x chunk holds a segment for exact_segments
    if (once && ns > 0) special = convert_x<NC>(A, wh.x, s0 * kStep, ns * kSegs, lane, xs, xf);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();

    for (int it = 0; tile < A.tiles; ++it) {
        const int64_t ntile = tile + gridDim.x;
        const bool has_n = ntile < A.tiles;
        Row nrow{};
        if (has_n) nrow = row_of<DT, 1>(A, ntile, wh.w_off, r, part, fn);

        float acc[1][NC];
#pragma unroll
        for (int n = 0; n < NC; ++n) acc[0][n] = 0.0f;
        for (int k = 0; k < ns; ++k) {
            if (!once && k % cs == 0) {
                // a new x chunk: steps [k, k + cs) of this wave
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                special = convert_x<NC>(A, wh.x, (s0 + k) * kStep, min(cs, ns - k) * kSegs, lane, xs, xf);
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                __builtin_amdgcn_wave_barrier();
            }
            Raw nxt[1];
            if (k + 1 < ns) {
                nxt[0] = f[0].load(s0 + k + 1);
            } else if (has_n) {
                nxt[0] = fn[0].load(s0);
            }
            const XView xv{xs, xf, zpad, min(cs, ns - (k / cs) * cs) * kSegs};
            step_mfma<DT, 1, NC>(f, cur, al, (k % cs) * kSegs, xv, acc);
            if (special) exact_segments<DT, 1, NC>(A, wh, row, r, part, xv, (k % cs) * kSegs, kSegs, (s0 + k) * kStep, acc);
            cur[0] = nxt[0];
        }
        reduce_store<1, NC, W>(A, wh, row, acc, red + (it & 1) * (W * NC * 16), tid);
        tile = ntile;
        row = nrow;
        f[0] = fn[0];
    }
}

// ---- several columns: the columns share each MFMA ---------------------------------------------------
//
// For N = 2..8 the columns go into the rows of the MFMA's A operand, so each weight code is
// unpacked once for all of them. This needs every MFMA to span few scale groups: the lane parts
// are mapped so that parts {0, 1} of an MFMA lie in one scale group and parts {2, 3} in one other
// (G = 2: Q4_0, Q8_0, Q4_K), or each part in its own 16-element group (G = 4: Q6_K). Rows 4w ..
// 4w + 2 of A (window w) hold the three x planes of one (column, group): G = 2: window 2c + g =
// column c of the set (2 columns per MFMA set), group g; G = 4: window g of the set's one column.
// A window holds its column's planes only at the k positions of its group (zeros elsewhere), so
// window w of D is that column's integer dot product over that group alone. Lane (r, p) receives
// window p of D, scales it with its group's block scale and x-segment factor, and accumulates it
// for its column; the parts of one column are added at the end (parts p and p ^ 1 for G = 2, all
// four for G = 4).
//
// Per format, for MFMA t = 0..3 of a step and lane part p: the segment (32 elements of the step)
// and 16-byte half that part p supplies, the group it belongs to, and the flush of the lane's D.

template <int DT> struct FmtN;

// Q4_K: part p loads units p and p + 4 of the block's 8 (16 bytes each): MFMA 0 / 1 take the low
// / high nibbles of unit p, MFMA 2 / 3 those of unit p + 4. Unit u holds chunk u / 2, half u % 2:
// its low nibbles are sub-block 2 (u / 2), its high nibbles sub-block 2 (u / 2) + 1. So MFMA t,
// group g (= p / 2) is sub-block 4 (t / 2) + t % 2 + 2 g, elements 16 (p % 2) .. +15 of it.
template <>
struct FmtN<Q4_K> {
    static constexpr int G = 2;
    struct Raw {
        uint4 qa, qb, hd;
    };
    const uint8_t * w;
    uint32_t qo, ho, u;
    int p;
    __device__ void init(const uint8_t * w_, int64_t M, int64_t nb, int64_t g0, int rs, int lr, int part) {
        w = w_;
        p = part;
        u = (uint32_t) rs * 16;
        qo = (uint32_t) (g0 * nb * 128 + lr * 16) + (uint32_t) p * u;
        ho = (uint32_t) (M * nb * 128 + g0 * nb * 16 + lr * 16);
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        const uint32_t q = __umul24((uint32_t) step * 8, u) + qo;
        r.qa = load16(w + q);
        r.qb = load16(w + q + 4 * u);
        r.hd = load16(w + (__umul24((uint32_t) step, u) + ho));
        return r;
    }
    __device__ static v4i bop(const Raw & r, int t) {
        return t == 0 ? lo4(r.qa) : t == 1 ? hi4(r.qa) : t == 2 ? lo4(r.qb) : hi4(r.qb);
    }
    __device__ static int seg(int t, int g) {
        return 4 * (t >> 1) + (t & 1) + 2 * g;
    }
    // the factors of the lane's window group (p % 2) in MFMA t: d * sc, -dmin * m
    // (get_scale_min_k4 of sub-block seg(t, p % 2))
    struct Sc {
        float k, o;
    };
    __device__ Sc scales(const Raw & r, int t, const uint32_t (&)[2]) const {
        const float d = half_bits(r.hd.x), dmin = half_bits(r.hd.x >> 16);
        const int s = seg(t, p & 1);
        const uint32_t s0 = r.hd.y, s1 = r.hd.z, s2 = r.hd.w;
        const int sh = 8 * (s & 3);
        float sc, m;
        if (s < 4) {
            sc = (float) ((s0 >> sh) & 63u);
            m = (float) ((s1 >> sh) & 63u);
        } else {
            const uint32_t t0 = s2 >> sh;
            sc = (float) ((t0 & 0x0Fu) | (((s0 >> sh) >> 2) & 0x30u));
            m = (float) (((t0 >> 4) & 0x0Fu) | (((s1 >> sh) >> 2) & 0x30u));
        }
        return Sc{d * sc, -dmin * m};
    }
    __device__ float apply(const Sc & c, int t, const v4i & D, const float4 * xf) const {
        const float4 f = xf[seg(t, p & 1)];
        return fmaf(c.k * f.x, planes(D), c.o * f.w);
    }
};

// Q4_0: MFMA t, group g is block 2t + g; part p supplies nibble half p % 2 (elements 16 (p % 2)
// .. +15) of block 2t + p / 2. Part p loads those 4 blocks' units and scales; the scale of its
// window's group p % 2 is its own (p / 2 == p % 2) or comes from lane + 32 (part p ^ 2).
template <>
struct FmtN<Q4_0> {
    static constexpr int G = 2;
    struct Raw {
        uint4 q[4];
        uint32_t d[2]; // own blocks' scales (t = 0, 1 | t = 2, 3 as 16-bit halves)
    };
    const uint8_t * w;
    uint32_t qo, dof, u, nb;
    int p;
    __device__ void init(const uint8_t * w_, int64_t M, int64_t nb_, int64_t g0, int rs, int lr, int part) {
        w = w_;
        p = part;
        nb = (uint32_t) nb_;
        u = (uint32_t) rs * 16;
        qo = (uint32_t) (g0 * nb_ * 16 + lr * 16);
        dof = (uint32_t) (M * nb_ * 16 + g0 * nb_ * 2 + lr * 2);
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        uint32_t dh[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t b = (uint32_t) step * 8 + 2 * t + (p >> 1);
            const bool ok = b < nb;
            b = ok ? b : 0;
            r.q[t] = load16(w + (__umul24(b, u) + qo));
            const uint32_t d = load_half(w + (__umul24(b, u >> 3) + dof));
            dh[t] = ok ? d : 0u;
        }
        r.d[0] = dh[0] | (dh[1] << 16);
        r.d[1] = dh[2] | (dh[3] << 16);
        return r;
    }
    // the codes minus 8 as int8: (c + 0x78) ^ 0x80 per byte (no carries: c < 16)
    __device__ v4i bop(const Raw & r, int t) const {
        const uint4 q = r.q[t];
        const int sh = (p & 1) ? 4 : 0;
        return as_v4i(make_uint4((((q.x >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u, (((q.y >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u,
                                 (((q.z >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u, (((q.w >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u));
    }
    __device__ static int seg(int t, int g) {
        return 2 * t + g;
    }
    struct Sc {
        float k;
    };
    __device__ Sc scales(const Raw & r, int t, const uint32_t (&other)[2]) const {
        const uint32_t mine = r.d[t >> 1] >> (16 * (t & 1)), theirs = other[t >> 1] >> (16 * (t & 1));
        return Sc{half_bits((p >> 1) == (p & 1) ? mine : theirs)};
    }
    __device__ float apply(const Sc & c, int t, const v4i & D, const float4 * xf) const {
        return c.k * xf[seg(t, p & 1)].x * planes(D);
    }
};

// Q8_0: MFMA t, group g is block 2t + g; part p supplies half p % 2 of block 2t + p / 2. Scales
// as for Q4_0.
template <>
struct FmtN<Q8_0> {
    static constexpr int G = 2;
    struct Raw {
        uint4 q[4];
        uint32_t d[2];
    };
    const uint8_t * w;
    uint32_t qo, dof, u, nb;
    int p;
    __device__ void init(const uint8_t * w_, int64_t M, int64_t nb_, int64_t g0, int rs, int lr, int part) {
        w = w_;
        p = part;
        nb = (uint32_t) nb_;
        u = (uint32_t) rs * 16;
        qo = (uint32_t) (g0 * nb_ * 32 + lr * 16) + (uint32_t) (p & 1) * u;
        dof = (uint32_t) (M * nb_ * 32 + g0 * nb_ * 2 + lr * 2);
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        uint32_t dh[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t b = (uint32_t) step * 8 + 2 * t + (p >> 1);
            const bool ok = b < nb;
            b = ok ? b : 0;
            r.q[t] = load16(w + (__umul24(2 * b, u) + qo));
            const uint32_t d = load_half(w + (__umul24(b, u >> 3) + dof));
            dh[t] = ok ? d : 0u;
        }
        r.d[0] = dh[0] | (dh[1] << 16);
        r.d[1] = dh[2] | (dh[3] << 16);
        return r;
    }
    __device__ v4i bop(const Raw & r, int t) const {
        const uint4 q = r.q[t];
        return as_v4i(make_uint4(q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u));
    }
    __device__ static int seg(int t, int g) {
        return 2 * t + g;
    }
    struct Sc {
        float k;
    };
    __device__ Sc scales(const Raw & r, int t, const uint32_t (&other)[2]) const {
        const uint32_t mine = r.d[t >> 1] >> (16 * (t & 1)), theirs = other[t >> 1] >> (16 * (t & 1));
        return Sc{half_bits((p >> 1) == (p & 1) ? mine : theirs)};
    }
    __device__ float apply(const Sc & c, int t, const v4i & D, const float4 * xf) const {
        return c.k * xf[seg(t, p & 1)].x * planes(D);
    }
};

// Q6_K: the single-column mapping (part p = task (h, hf) = (p / 2, p % 2): elements
// 128 h + 32 t + 16 hf + i in MFMA t), each part its own 16-element group (G = 4), which is also
// its window.
template <>
struct FmtN<Q6_K> : Fmt<Q6_K> {
    static constexpr int G = 4;
    __device__ static int seg(int t, int g) { // the segment of group (task) g in MFMA t
        return 4 * (g >> 1) + t;
    }
    // the 6-bit codes minus 32 as int8: (c + 0x60) ^ 0x80 per byte (no carries: c < 64)
    __device__ static v4i bop(const Raw & r, int t) {
        const v4i b = Fmt<Q6_K>::bop(r, t);
        return as_v4i(make_uint4(((uint32_t) b.x + 0x60606060u) ^ 0x80808080u, ((uint32_t) b.y + 0x60606060u) ^ 0x80808080u,
                                 ((uint32_t) b.z + 0x60606060u) ^ 0x80808080u, ((uint32_t) b.w + 0x60606060u) ^ 0x80808080u));
    }
    // d * scale of the lane's group p in MFMA t (scale index 8 h + 2 t + hf, stored xor 0x80)
    struct Sc {
        float k;
    };
    __device__ Sc scales(const Raw & r, int t, const uint32_t (&)[2]) const {
        const int h = p >> 1, hf = p & 1;
        const uint32_t sw = h ? (t < 2 ? r.sc.z : r.sc.w) : (t < 2 ? r.sc.x : r.sc.y);
        return Sc{half_bits(r.d) * ((float) ((sw >> (8 * (2 * (t & 1) + hf))) & 0xFFu) - 128.0f)};
    }
    __device__ float apply(const Sc & c, int t, const v4i & D, const float4 * xf) const {
        return c.k * xf[seg(t, p)].x * planes(D);
    }
};

// The lane's A operand for MFMA t of set s: byte offset inside its column's XSeg run of the step,
// the column, or -1 (zeros). Row i = l % 16 = 4 w + k (window w, plane k), part p = l / 16.
template <int DT, int NC>
struct ALaneN {
    static constexpr int G = FmtN<DT>::G;
    static constexpr int CPS = G == 2 ? 2 : 1; // columns per MFMA set
    static constexpr int NS = (NC + CPS - 1) / CPS;
    int off[NS][4];
    int col[NS];
    __device__ explicit ALaneN(int lane) {
        const int i = lane & 15, p = lane >> 4;
        const int w = i >> 2, k = i & 3;
        const int c = G == 2 ? w >> 1 : 0, g = G == 2 ? (w & 1) : w;
        const int pg = G == 2 ? p >> 1 : p; // the group of part p
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int n = s * CPS + c;
            col[s] = n;
#pragma unroll
            for (int t = 0; t < 4; ++t)
                off[s][t] = (k < 3 && g == pg && n < NC) ? FmtN<DT>::seg(t, pg) * kSegBytes + k * 32 + (p & 1) * 16 : -1;
        }
    }
};

// the column whose partial lane part p holds in set s
template <int DT, int NC>
__device__ __forceinline__ int lane_col(int s, int p) {
    return s * ALaneN<DT, NC>::CPS + (FmtN<DT>::G == 2 ? p >> 1 : 0);
}

// one step of NC columns: acc[s] is the lane's partial of column lane_col(s, p)
// (sets S0 .. S1 only; column n's x sits in slot n - c0 of the view)
template <int DT, int NC, int S0 = 0, int S1 = ALaneN<DT, NC>::NS>
__device__ __forceinline__ void step_mfma_n(const FmtN<DT> & f, const typename FmtN<DT>::Raw & raw, const ALaneN<DT, NC> & al, int sg0,
                                            const XView & xv, float (&acc)[ALaneN<DT, NC>::NS], int lane, int c0 = 0) {
    const int p = lane >> 4;
    uint32_t other[2] = {0u, 0u};
    if constexpr (DT == Q4_0 || DT == Q8_0) {
        other[0] = __shfl_xor(raw.d[0], 32);
        other[1] = __shfl_xor(raw.d[1], 32);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const v4i B = f.bop(raw, t);
        const typename FmtN<DT>::Sc sc = f.scales(raw, t, other);
#pragma unroll
        for (int s = S0; s < S1; ++s) {
            const int n = al.col[s];
            const uint8_t * base = reinterpret_cast<const uint8_t *>(xv.xs + (n < NC ? n - c0 : 0) * xv.nseg + sg0);
            const uint8_t * pa = al.off[s][t] >= 0 ? base + al.off[s][t] : xv.zpad;
            const v4i A = *reinterpret_cast<const v4i *>(pa);
            const v4i D = mfma(A, B, v4i{0, 0, 0, 0});
            const int nl = lane_col<DT, NC>(s, p);
            if (nl < NC) acc[s] += f.apply(sc, t, D, xv.xf + (nl - c0) * xv.nseg + sg0);
        }
    }
}

// the parts of one column: G = 2: parts p and p ^ 1; G = 4: all four. True on the lane that
// stores the column's sum (window 0 of it)
template <int DT>
__device__ __forceinline__ bool add_parts(float & v, int p) {
    v += __shfl_xor(v, 16);
    if constexpr (FmtN<DT>::G == 4) v += __shfl_xor(v, 32);
    return FmtN<DT>::G == 2 ? (p & 1) == 0 : p == 0;
}

// columns-in-rows lane mapping (k_mvn, k_mvc): for the columns c0 .. c1 - 1 held in slots
// n - c0 of the view, the exact sums of the flagged segments sg .. sg + cnt - 1 (segment sg + g
// starts at element k0 + 32 g; column n's x at x + n x_s1) go into the partial of the lane that
// stores column n
template <int DT, int NC>
__device__ void exact_segments_n(const R32Row & row, const float * x, int64_t x_s1, const XView & xv, int sg, int cnt, int64_t k0, int c0, int c1,
                                 float (&acc)[ALaneN<DT, NC>::NS], int p) {
    constexpr int CPS = ALaneN<DT, NC>::CPS;
#pragma unroll
    for (int n = 0; n < NC; ++n) {
        if (n < c0 || n >= c1) continue;
        for (int g = 0; g < cnt; ++g) {
            if (!flagged_at(xv.xf + (n - c0) * xv.nseg, sg + g)) continue;
            const float e = seg_exact<DT>(row, x + n * x_s1, k0 + 32 * (int64_t) g, p);
            const bool mine = FmtN<DT>::G == 2 ? p == 2 * (n % CPS) : p == 0;
            if (mine) acc[n / CPS] += e;
        }
    }
}

// Streaming form for N = 2..8 with the columns in the MFMA's A rows (see above); otherwise as
// k_mvs: a persistent grid of 16-row tiles, x converted once per wave (when its range fits the
// LDS budget), the next step's loads in flight while the current one is computed.
template <int DT, int NC, int W>
__global__ __launch_bounds__(64 * W) void k_mvn(MvArgs A) {
    using F = FmtN<DT>;
    using Raw = typename F::Raw;
    using AL = ALaneN<DT, NC>;
    constexpr int G = F::G, CPS = AL::CPS, NS = AL::NS;
    extern __shared__ uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, part = lane >> 4;
    const Where wh = where_of(A);

    const int64_t s0 = A.nst * wave / W, s1 = A.nst * (wave + 1) / W;
    const int ns = (int) (s1 - s0);
    const int cs = A.cs;
    const bool once = cs >= ns;
    XSeg * xs = reinterpret_cast<XSeg *>(lds) + (size_t) wave * cs * kSegs * NC;
    float4 * xf = reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * cs * kSegs * NC) + (size_t) wave * cs * kSegs * NC;
    float * red = reinterpret_cast<float *>(reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * cs * kSegs * NC) +
                                            (size_t) W * cs * kSegs * NC); // [2][W][NC][16]
    uint8_t * zpad = reinterpret_cast<uint8_t *>(red + 2 * W * NC * 16);
    if (lane < 4) reinterpret_cast<uint32_t *>(zpad)[lane] = 0u;
    const AL al(lane);

    int64_t tile = blockIdx.x;
    F f, fn;
    Row row;
    {
        const int j = tile >= A.tstart[1] ? (tile >= A.tstart[2] ? 2 : 1) : 0;
        row = Row{j, A.M[j], (tile - A.tstart[j]) * 16};
        const int64_t m = min(row.m0 + r, row.M - 1), g0 = m & ~(int64_t) 31;
        f.init(A.w[j] + wh.w_off, row.M, A.nb, g0, (int) min<int64_t>(32, row.M - g0), (int) (m - g0), part);
    }
    Raw cur;
    if (ns > 0) cur = f.load(s0);
    bool special = false; // the current x chunk holds a segment for exact_segments_n
    if (once && ns > 0) special = convert_x<NC>(A, wh.x, s0 * kStep, ns * kSegs, lane, xs, xf);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();

    for (int it = 0; tile < A.tiles; ++it) {
        const int64_t ntile = tile + gridDim.x;
        const bool has_n = ntile < A.tiles;
        Row nrow{};
        if (has_n) {
            const int j = ntile >= A.tstart[1] ? (ntile >= A.tstart[2] ? 2 : 1) : 0;
            nrow = Row{j, A.M[j], (ntile - A.tstart[j]) * 16};
            const int64_t m = min(nrow.m0 + r, nrow.M - 1), g0 = m & ~(int64_t) 31;
            fn.init(A.w[j] + wh.w_off, nrow.M, A.nb, g0, (int) min<int64_t>(32, nrow.M - g0), (int) (m - g0), part);
        }
        float acc[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) acc[s] = 0.0f;
        for (int k = 0; k < ns; ++k) {
            if (!once && k % cs == 0) {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                special = convert_x<NC>(A, wh.x, (s0 + k) * kStep, min(cs, ns - k) * kSegs, lane, xs, xf);
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                __builtin_amdgcn_wave_barrier();
            }
            Raw nxt;
            if (k + 1 < ns) {
                nxt = f.load(s0 + k + 1);
            } else if (has_n) {
                nxt = fn.load(s0);
            }
            const XView xv{xs, xf, zpad, min(cs, ns - (k / cs) * cs) * kSegs};
            step_mfma_n<DT, NC>(f, cur, al, (k % cs) * kSegs, xv, acc, lane);
            if (special)
                exact_segments_n<DT, NC>(r32_row(A.w[row.j] + wh.w_off, row.M, A.nb, row.m0 + r), wh.x, A.x_s1, xv, (k % cs) * kSegs, kSegs,
                                         (s0 + k) * kStep, 0, NC, acc, part);
            cur = nxt;
        }
        // the parts of a column (add_parts), then the waves through LDS
        float * rb = red + (it & 1) * (W * NC * 16);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            float v = acc[s];
            const bool st = add_parts<DT>(v, part);
            const int n = lane_col<DT, NC>(s, part);
            if (n < NC && st) rb[(wave * NC + n) * 16 + r] = v;
        }
        __syncthreads();
        if (tid < NC * 16) {
            const int n = tid / 16, rr = tid % 16;
            const int64_t m = row.m0 + rr;
            if (m < row.M) {
                float v = 0.0f;
#pragma unroll
                for (int w2 = 0; w2 < W; ++w2) v += rb[(w2 * NC + n) * 16 + rr];
                A.y[row.j][wh.y_off + n * A.ys1[row.j] + m] = v;
            }
        }
        tile = ntile;
        row = nrow;
        f = fn;
    }
}

template <int DT>
void * pick_columns(int nc) {
    switch (nc) {
        case 2: return (void *) k_mvn<DT, 2, 4>;
        case 3: return (void *) k_mvn<DT, 3, 4>;
        case 4: return (void *) k_mvn<DT, 4, 4>;
        case 5: return (void *) k_mvn<DT, 5, 4>;
        case 6: return (void *) k_mvn<DT, 6, 4>;
        case 7: return (void *) k_mvn<DT, 7, 4>;
        default: return (void *) k_mvn<DT, 8, 4>;
    }
}

// ---- several columns, one tile per work-group (the form for N = 2..8, one slice) -----------------
//
// x goes through a pre-pass first (k_x_planes: every 32-element segment of every column as its
// two int8 planes and factors, in scratch), so the matvec work-groups only copy their part of it
// into LDS. A work-group owns 16 rows and one K chunk of 16 steps (4096 elements): its 8 waves take
// 2 steps each and issue all their loads at once (x planes first, then weights), like the
// one-column burst form. With several chunks the work-groups write partial sums, and the last
// chunk of a row tile to finish (arrival counters cleared by the pre-pass) adds them in chunk order.

constexpr int kMcW = 8, kMcSpw = 2, kMcChunk = kMcW * kMcSpw; // waves, steps per wave, steps per chunk

struct McArgs {
    const uint8_t * w[3];
    int64_t M[3];
    float * y[3];
    int64_t ys1[3];
    int64_t tstart[4];   // matrix j owns row tiles [tstart[j], tstart[j + 1])
    int64_t nb, nst, nchunks;
    const XSeg * planes; // [NC][nsegp]
    const float4 * fac;  // [NC][nsegp]
    int64_t nsegp;       // segments per column in the scratch (nchunks * 128)
    float * part;        // nchunks > 1: [nchunks][NC][tiles * 16]
    uint32_t * arrive;   // nchunks > 1: chunks done per row tile (zeroed by k_x_planes)
    int64_t prow;        // tiles * 16
    const float * x;     // !PRE: x itself (columns x_s1 floats apart, 16-byte aligned), K elements
    int64_t x_s1, K;
};

// one work-group per 16 x 32 = 512 elements... (64 threads: 16 segments, 4 lanes each)
__global__ __launch_bounds__(64) void k_x_planes(const float * x, int64_t x_s1, int64_t K, int64_t nsegp, XSeg * planes, float4 * fac,
                                                 uint32_t * arrive, int64_t narrive) {
    const int lane = threadIdx.x, q = lane & 3;
    // the K-chunk arrival counters of the matvec that follows start at zero
    for (int64_t i = ((int64_t) blockIdx.y * gridDim.x + blockIdx.x) * 64 + lane; i < narrive; i += (int64_t) gridDim.x * gridDim.y * 64) arrive[i] = 0u;
    const int64_t n = blockIdx.y;
    const int64_t g = (int64_t) blockIdx.x * 16 + (lane >> 2);
    const int64_t e = 32 * g + 8 * q;
    float v[8];
    const float * xp = x + n * x_s1 + e;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = e < K ? xp[i] : 0.0f;
    // convert_seg writes segment (lane >> 2) of the 16 starting at this block's first
    convert_seg(v, lane >> 2, 16, q, planes + n * nsegp + (int64_t) blockIdx.x * 16, fac + n * nsegp + (int64_t) blockIdx.x * 16);
}

// PRE: x comes converted from k_x_planes; else each wave converts its own range of x here (after
// issuing its weight loads), which saves the pre-pass launch where the columns are few
// 4 waves per SIMD (two work-groups per CU) where that fits without spilling
constexpr int mc_waves(int dt, int nc) {
    return (dt == Q4_K && nc >= 7) || (dt == Q6_K && nc >= 5) ? 3 : 4;
}

template <int DT, int NC, bool PRE>
__global__ __launch_bounds__(64 * kMcW) __attribute__((amdgpu_waves_per_eu(mc_waves(DT, NC), 8))) void k_mvc(McArgs A) {
    using F = FmtN<DT>;
    using Raw = typename F::Raw;
    using AL = ALaneN<DT, NC>;
    constexpr int CPS = AL::CPS, NS = AL::NS, W = kMcW, SPW = kMcSpw, SEGS = SPW * kSegs;
    extern __shared__ uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, part = lane >> 4;
    const int64_t rt = blockIdx.x;
    const int c = (int) blockIdx.y;
    const int64_t sb = (int64_t) c * kMcChunk + wave * SPW;
    const int ns = (int) max<int64_t>(0, min<int64_t>(SPW, A.nst - sb));

    // x planes of the wave's 2 steps for every column (the scratch holds whole chunks, zero past K)
    // (plain scalars: arrays of vector types end up in scratch memory). x of the first pass of
    // columns now, ahead of the weights; the second pass's (NC > 4) once the first is in LDS
    constexpr int PC = NC < 4 ? NC : 4, NP = (NC + 3) / 4;
    uint32_t xq[PC][6]; // the 16 segments' 1536 plane bytes: 16 per lane, then 8 per lane
    float xfq[PC][4];
    float xe[PC][8];
    const int64_t e = sb * kStep + 32 * (lane >> 2) + 8 * (lane & 3); // !PRE: lane's 8 elements
    const bool xok = e < A.K && (lane >> 2) < ns * kSegs;
    auto load_x = [&](int c0) {
#pragma unroll
        for (int k = 0; k < PC; ++k) {
            const int n = c0 + k < NC ? c0 + k : c0; // (a column past NC re-reads the pass's first)
            if constexpr (PRE) {
                const uint8_t * pb = reinterpret_cast<const uint8_t *>(A.planes + n * A.nsegp + sb * kSegs);
                const uint4 q = reinterpret_cast<const uint4 *>(pb)[lane];
                const uint2 q2 = reinterpret_cast<const uint2 *>(pb + 1024)[lane];
                const float4 fq = A.fac[n * A.nsegp + sb * kSegs + (lane & 15)];
                xq[k][0] = q.x; xq[k][1] = q.y; xq[k][2] = q.z; xq[k][3] = q.w; xq[k][4] = q2.x; xq[k][5] = q2.y;
                xfq[k][0] = fq.x; xfq[k][1] = fq.y; xfq[k][2] = fq.z; xfq[k][3] = fq.w;
            } else {
                // branch-free: past K (or past the wave's steps) re-read element 0 and drop it
                const float * xp = A.x + n * A.x_s1 + (xok ? e : 0);
                const float4 u = *reinterpret_cast<const float4 *>(xp);
                const float4 w = *reinterpret_cast<const float4 *>(xp + 4);
                xe[k][0] = xok ? u.x : 0.0f; xe[k][1] = xok ? u.y : 0.0f; xe[k][2] = xok ? u.z : 0.0f; xe[k][3] = xok ? u.w : 0.0f;
                xe[k][4] = xok ? w.x : 0.0f; xe[k][5] = xok ? w.y : 0.0f; xe[k][6] = xok ? w.z : 0.0f; xe[k][7] = xok ? w.w : 0.0f;
            }
        }
    };
    load_x(0);
    __builtin_amdgcn_sched_barrier(0);
    const int j = rt >= A.tstart[1] ? (rt >= A.tstart[2] ? 2 : 1) : 0;
    const int64_t M = A.M[j], m0 = (rt - A.tstart[j]) * 16;
    F f;
    {
        const int64_t m = min(m0 + r, M - 1), g0 = m & ~(int64_t) 31;
        f.init(A.w[j], M, A.nb, g0, (int) min<int64_t>(32, M - g0), (int) (m - g0), part);
    }
    Raw buf[SPW];
#pragma unroll
    for (int s = 0; s < SPW; ++s) buf[s] = f.load(s < ns ? sb + s : (ns > 0 ? sb : 0));
    __builtin_amdgcn_sched_barrier(0);

    // LDS holds PC columns' x at a time: columns go through it in passes of up to 4 (the
    // weights stay in registers), so that NC = 5..8 still leaves room for two work-groups per CU
    XSeg * xs = reinterpret_cast<XSeg *>(lds) + (size_t) wave * PC * SEGS;
    float4 * xf = reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * PC * SEGS) + (size_t) wave * PC * SEGS;
    float * red = reinterpret_cast<float *>(reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * PC * SEGS) + (size_t) W * PC * SEGS);
    uint8_t * zpad = reinterpret_cast<uint8_t *>(red + W * NC * 16);
    if (tid < 4) reinterpret_cast<uint32_t *>(zpad)[tid] = 0u;
    __syncthreads(); // (zpad is written by wave 0 for all)

    const AL al(lane);
    const XView xv{xs, xf, zpad, SEGS};
    float acc[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) acc[s] = 0.0f;
    // flagged x segments of column n: bit g (PRE) or 4 g of fmask[n] (scalar)
    uint64_t fmask[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) fmask[n] = 0;
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        if (q > 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
#pragma unroll
        for (int k = 0; k < PC; ++k) {
            if (4 * q + k < NC) {
                if constexpr (PRE) {
                    uint8_t * xb = reinterpret_cast<uint8_t *>(xs + k * SEGS);
                    reinterpret_cast<uint4 *>(xb)[lane] = make_uint4(xq[k][0], xq[k][1], xq[k][2], xq[k][3]);
                    reinterpret_cast<uint2 *>(xb + 1024)[lane] = make_uint2(xq[k][4], xq[k][5]);
                    if (lane < 16) xf[k * SEGS + lane] = make_float4(xfq[k][0], xfq[k][1], xfq[k][2], xfq[k][3]);
                    fmask[4 * q + k] = __ballot(lane < 16 && __float_as_uint(xfq[k][0]) == 0x80000000u);
                } else {
                    fmask[4 * q + k] = __ballot(convert_seg(xe[k], lane >> 2, SEGS, lane & 3, xs + k * SEGS, xf + k * SEGS));
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (q + 1 < NP) load_x(4 * (q + 1)); // the next pass's x, in flight during this pass
        // pass q: the sets of columns 4q .. 4q + 3
#pragma unroll
        for (int s = 0; s < SPW; ++s) {
            if (s < ns) {
                if (q == 0) step_mfma_n<DT, NC, 0, (4 / CPS < NS ? 4 / CPS : NS)>(f, buf[s], al, s * kSegs, xv, acc, lane, 0);
                else step_mfma_n<DT, NC, (4 / CPS < NS ? 4 / CPS : NS), NS>(f, buf[s], al, s * kSegs, xv, acc, lane, 4);
            }
        }
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        float v = acc[s];
        const bool st = add_parts<DT>(v, part);
        const int n = lane_col<DT, NC>(s, part);
        if (n < NC && st) red[(wave * NC + n) * 16 + r] = v;
    }
    // the exact sums of flagged x segments (with no accumulator live any more)
    for (int n = 0; n < NC; ++n) {
        if (fmask[n] != 0)
            exact_red_n<DT>(A.w[j], M, A.nb, m0, A.x + n * A.x_s1, fmask[n], PRE ? 1 : 4, ns * kSegs, sb * kStep, red + (wave * NC + n) * 16);
    }
    __syncthreads();
    if (tid < NC * 16) {
        const int n = tid / 16, rr = tid % 16;
        float v = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < W; ++w2) v += red[(w2 * NC + n) * 16 + rr];
        if (A.nchunks == 1) {
            if (m0 + rr < M) A.y[j][n * A.ys1[j] + m0 + rr] = v;
        } else {
            // the chunk's partial sums, visible to every XCD before the row tile's count moves
            // (agent-scope stores write through the L2; then wait for them)
            __hip_atomic_store(A.part + ((int64_t) c * NC + n) * A.prow + rt * 16 + rr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (A.nchunks == 1) return;
    __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): this wave's partial-sum stores are done
    __syncthreads();
    // (in the dynamic LDS after zpad: a static __shared__ would shift the dynamic block off its
    // 16-byte alignment)
    // the count moves after every storing wave's write-through stores are acknowledged (their
    // vmcnt(0), then the barrier): the ordering a release would give, without its L2 write-back
    uint32_t & last = *reinterpret_cast<uint32_t *>(zpad + 16);
    if (tid == 0) last = __hip_atomic_fetch_add(A.arrive + rt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t) A.nchunks - 1;
    __syncthreads();
    // the last chunk of the row tile to finish adds all of them, in chunk order (agent-scope
    // loads: the other chunks' sums may come from other XCDs)
    if (last && tid < NC * 16) {
        const int n = tid / 16, rr = tid % 16;
        if (m0 + rr < M) {
            A.y[j][n * A.ys1[j] + m0 + rr] = ordered_sum(A.part + n * A.prow + rt * 16 + rr, NC * A.prow, A.nchunks);
        }
    }
}

// ---- several columns on 32 x 32 x 32 MFMAs: k_mvw ------------------------------------------------
//
// v_mfma_i32_32x32x32_i8 takes the codes of a whole R32 group (32 rows: column j of B) over 32
// consecutive elements of K (lane (j, h) supplies the 16 codes of k-half h, one 16-byte R32 unit
// or the nibbles of one), and x in its 32 A rows: row 4c + k = plane k of column c (k < 3; row
// 4c + 3 is zero). One MFMA covers one 32-element scale group of Q4_0 / Q8_0 / Q4_K for up to 8
// columns, so no A row is zero-padded by group and every code is unpacked once for all columns.
// Q6_K's groups are 16 elements: its A rows are (column c, group s, plane k) at 4 (2c + s) + k,
// holding x only in k-half s, for 4 columns per MFMA. Lane (j, h) receives D rows 8 (i / 4) + 4h +
// i % 4: column 2 (i / 4) + h's three planes (Q6_K: column i / 4's, group h), which it scales with
// its row's group factor and the segment's x factor. A work-group owns one 32-row tile and one K
// chunk of kMwW x kMwSpw steps; every wave issues all its loads at once (x first), and the waves'
// sums meet in LDS in wave order; chunks meet as in k_mvc.

typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16i mfma32(v4i a, v4i b) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0}, 0, 0, 0);
}

// Per format: init() resolves the lane's row (r < rs of the R32 group at g0) as 32-bit byte offsets
// from the slice base; load(step) fetches the lane's bytes of one step; for MFMA q of the step
// (Q = 8 per step), seg(q) is the x segment, bop(raw, q) the B operand (16 int8 codes of k-half
// h), and fac(raw, q) the group's factors {scale, offset} (offset multiplies the segment's x sum).
template <int DT> struct FmtW;

// Q8_0: MFMA q = block q of the step; lane half h: unit 2q + h (bytes xor 0x80 stored)
template <>
struct FmtW<Q8_0> {
    static constexpr bool OFF = false;
    struct Raw {
        uint4 u[8];
        uint32_t d[4];
    };
    const uint8_t * w;
    uint32_t qo, dof, u, nb;
    __device__ void init(const uint8_t * w_, int64_t M, int64_t nb_, int64_t g0, int rs, int lr, int h) {
        w = w_;
        nb = (uint32_t) nb_;
        u = (uint32_t) rs * 16;
        qo = (uint32_t) (g0 * nb_ * 32 + lr * 16) + (uint32_t) h * u;
        dof = (uint32_t) (M * nb_ * 32 + g0 * nb_ * 2 + lr * 2);
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        uint32_t dh[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            uint32_t b = (uint32_t) step * 8 + q;
            const bool ok = b < nb;
            b = ok ? b : 0;
            r.u[q] = load16(w + (__umul24(2 * b, u) + qo));
            const uint32_t d = load_half(w + (__umul24(b, u >> 3) + dof));
            dh[q] = ok ? d : 0u;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) r.d[i] = dh[2 * i] | (dh[2 * i + 1] << 16);
        return r;
    }
    __device__ static int seg(int q) {
        return q;
    }
    __device__ static v4i bop(const Raw & r, int q) {
        const uint4 v = r.u[q];
        return as_v4i(make_uint4(v.x ^ 0x80808080u, v.y ^ 0x80808080u, v.z ^ 0x80808080u, v.w ^ 0x80808080u));
    }
    __device__ static float2 fac(const Raw & r, int q) {
        return make_float2(half_bits(r.d[q >> 1] >> (16 * (q & 1))), 0.0f);
    }
};

// Q4_0: MFMA q = block q; lane half h: the low (h = 0: elements 0..15) or high nibbles of the
// block's one unit, minus 8
template <>
struct FmtW<Q4_0> {
    static constexpr bool OFF = false;
    struct Raw {
        uint4 u[8];
        uint32_t d[4];
    };
    const uint8_t * w;
    uint32_t qo, dof, u, nb;
    int h;
    __device__ void init(const uint8_t * w_, int64_t M, int64_t nb_, int64_t g0, int rs, int lr, int h_) {
        w = w_;
        h = h_;
        nb = (uint32_t) nb_;
        u = (uint32_t) rs * 16;
        qo = (uint32_t) (g0 * nb_ * 16 + lr * 16);
        dof = (uint32_t) (M * nb_ * 16 + g0 * nb_ * 2 + lr * 2);
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        uint32_t dh[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            uint32_t b = (uint32_t) step * 8 + q;
            const bool ok = b < nb;
            b = ok ? b : 0;
            r.u[q] = load16(w + (__umul24(b, u) + qo));
            const uint32_t d = load_half(w + (__umul24(b, u >> 3) + dof));
            dh[q] = ok ? d : 0u;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) r.d[i] = dh[2 * i] | (dh[2 * i + 1] << 16);
        return r;
    }
    __device__ static int seg(int q) {
        return q;
    }
    __device__ v4i bop(const Raw & r, int q) const {
        const uint4 v = r.u[q];
        const int sh = 4 * h;
        return as_v4i(make_uint4((((v.x >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u, (((v.y >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u,
                                 (((v.z >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u, (((v.w >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u));
    }
    __device__ static float2 fac(const Raw & r, int q) {
        return make_float2(half_bits(r.d[q >> 1] >> (16 * (q & 1))), 0.0f);
    }
};

// Q4_K: MFMA q = sub-block q of the block (the step); lane half h: unit 2 (q / 2) + h, low
// nibbles for even q (sub-block 2c), high for odd (2c + 1); factors d * sc, -dmin * m
template <>
struct FmtW<Q4_K> {
    static constexpr bool OFF = true;
    struct Raw {
        uint4 u[4], hd;
    };
    const uint8_t * w;
    uint32_t qo, ho, u;
    __device__ void init(const uint8_t * w_, int64_t M, int64_t nb, int64_t g0, int rs, int lr, int h) {
        w = w_;
        u = (uint32_t) rs * 16;
        qo = (uint32_t) (g0 * nb * 128 + lr * 16) + (uint32_t) h * u;
        ho = (uint32_t) (M * nb * 128 + g0 * nb * 16 + lr * 16);
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        const uint32_t q = __umul24((uint32_t) step * 8, u) + qo;
#pragma unroll
        for (int c = 0; c < 4; ++c) r.u[c] = load16(w + q + (uint32_t) (2 * c) * u);
        r.hd = load16(w + (__umul24((uint32_t) step, u) + ho));
        return r;
    }
    __device__ static int seg(int q) {
        return q;
    }
    __device__ static v4i bop(const Raw & r, int q) {
        return (q & 1) ? hi4(r.u[q >> 1]) : lo4(r.u[q >> 1]);
    }
    __device__ static float2 fac(const Raw & r, int s) {
        const float d = half_bits(r.hd.x), dmin = half_bits(r.hd.x >> 16);
        const uint32_t s0 = r.hd.y, s1 = r.hd.z, s2 = r.hd.w;
        const int sh = 8 * (s & 3);
        float sc, m;
        if (s < 4) {
            sc = (float) ((s0 >> sh) & 63u);
            m = (float) ((s1 >> sh) & 63u);
        } else {
            const uint32_t t0 = s2 >> sh;
            sc = (float) ((t0 & 0x0Fu) | (((s0 >> sh) >> 2) & 0x30u));
            m = (float) (((t0 >> 4) & 0x0Fu) | (((s1 >> sh) >> 2) & 0x30u));
        }
        return make_float2(d * sc, -dmin * m);
    }
};

// Q6_K: MFMA q = (half-block hh = q / 4, run t = q % 4): elements 128 hh + 32 t + 16 h + i of
// the block (segment 4 hh + t), lane half h = the 16-element group; codes from ql units
// 4 hh + h (t = 0, 2) / 4 hh + 2 + h (t = 1, 3), low nibbles for t < 2, with bits 2t, 2t + 1 of
// qh unit 8 + 2 hh + h on top, minus 32; factor d * scale[8 hh + 2t + h]
template <>
struct FmtW<Q6_K> {
    static constexpr bool OFF = false;
    struct Raw {
        uint4 qa[2], qc[2], qh[2], sc;
        uint32_t d;
    };
    const uint8_t * qb;
    const uint8_t * sb;
    const uint8_t * db;
    uint32_t qblk, qunit, sblk, dblk;
    int h;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb, int64_t g0, int rs, int lr, int h_) {
        h = h_;
        qb = w + (uint64_t) g0 * nb * 192 + (uint64_t) lr * 16;
        sb = w + (uint64_t) M * nb * 192 + (uint64_t) g0 * nb * 16 + (uint64_t) lr * 16;
        db = w + (uint64_t) M * nb * 208 + (uint64_t) g0 * nb * 2 + (uint64_t) lr * 2;
        qblk = (uint32_t) rs * 192;
        qunit = (uint32_t) rs * 16;
        sblk = (uint32_t) rs * 16;
        dblk = (uint32_t) rs * 2;
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        const uint8_t * b = qb + (uint32_t) step * qblk;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            r.qa[hh] = load16(b + (uint32_t) (4 * hh + h) * qunit);
            r.qc[hh] = load16(b + (uint32_t) (4 * hh + 2 + h) * qunit);
            r.qh[hh] = load16(b + (uint32_t) (8 + 2 * hh + h) * qunit);
        }
        r.sc = load16(sb + (uint32_t) step * sblk);
        r.d = load_half(db + (uint32_t) step * dblk);
        return r;
    }
    __device__ static int seg(int q) {
        return q;
    }
    __device__ static v4i bop(const Raw & r, int q) {
        const int hh = q >> 2, t = q & 3;
        const uint4 ql = (t & 1) ? r.qc[hh] : r.qa[hh];
        const uint4 qh = r.qh[hh];
        const int ls = t < 2 ? 0 : 4, hs = 2 * t;
        return as_v4i(make_uint4(((((ql.x >> ls) & 0x0F0F0F0Fu) | (((qh.x >> hs) << 4) & 0x30303030u)) + 0x60606060u) ^ 0x80808080u,
                                 ((((ql.y >> ls) & 0x0F0F0F0Fu) | (((qh.y >> hs) << 4) & 0x30303030u)) + 0x60606060u) ^ 0x80808080u,
                                 ((((ql.z >> ls) & 0x0F0F0F0Fu) | (((qh.z >> hs) << 4) & 0x30303030u)) + 0x60606060u) ^ 0x80808080u,
                                 ((((ql.w >> ls) & 0x0F0F0F0Fu) | (((qh.w >> hs) << 4) & 0x30303030u)) + 0x60606060u) ^ 0x80808080u));
    }
    __device__ float2 fac(const Raw & r, int q) const {
        const int hh = q >> 2, t = q & 3;
        // scale byte 8 hh + 2t + h (stored xor 0x80): word 2 hh + t / 2, byte 2 (t % 2) + h
        const uint32_t sw = hh ? (t < 2 ? r.sc.z : r.sc.w) : (t < 2 ? r.sc.x : r.sc.y);
        return make_float2(half_bits(r.d) * ((float) ((sw >> (8 * (2 * (t & 1) + h))) & 0xFFu) - 128.0f), 0.0f);
    }
};

// columns per MFMA set: 8 (32-element groups), 4 (Q6_K)
template <int DT>
constexpr int mw_cps() {
    return DT == Q6_K ? 4 : 8;
}

struct MwArgs {
    const uint8_t * w[3];
    int64_t M[3];
    float * y[3];
    int64_t ys1[3];
    int64_t tstart[4]; // matrix j owns row tiles [tstart[j], tstart[j + 1])
    int64_t nb, nst, K, nchunks;
    const float * x;   // columns x_s1 floats apart, 16-byte aligned
    int64_t x_s1;
    float * part;      // nchunks > 1: [nchunks][NC][prow] partial sums
    uint32_t * arrive; // nchunks > 1: chunks done per row tile, zero between launches
    int64_t prow;      // tiles * rows per tile
};

// Work-group: RW x KW waves; wave (rw, kw) takes rows 32 rw .. + 31 of the tile and steps
// 2 kw, 2 kw + 1 of the K chunk (2 KW steps); all of them share the chunk's x, converted once per
// work-group into LDS by all its threads while the weight loads are in flight.
template <int DT, int NC, int RW, int KW>
__global__ __launch_bounds__(64 * RW * KW) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_mvw(MwArgs A) {
    using F = FmtW<DT>;
    using Raw = typename F::Raw;
    constexpr int CPS = mw_cps<DT>(), NS = (NC + CPS - 1) / CPS, SPW = 2, CH = KW * SPW, SEGS = CH * kSegs, R = 32 * RW, T = 64 * RW * KW;
    extern __shared__ uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); // wave-uniform: scalar control
    const int rw = wave % RW, kw = wave / RW;
    const int r = lane & 31, h = lane >> 5;
    const int64_t rt = blockIdx.x;
    const int c = (int) blockIdx.y;
    const int64_t cb = (int64_t) c * CH;                      // the chunk's first step
    const int64_t sb = cb + kw * SPW;                         // the wave's first step
    const int ns = (int) max<int64_t>(0, min<int64_t>(SPW, A.nst - sb));

    // x of the chunk: thread t converts elements 8 (t % 4) .. + 7 of segment (t / 4) % SEGS of
    // column (t / 4) / SEGS (+ T / 4 / SEGS per pass); loads issued first, branch-free
    constexpr int TASKS = NC * SEGS * 4, PASSES = (TASKS + T - 1) / T;
    float xe[PASSES][8];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int task = p * T + tid, g = (task >> 2) % SEGS, n = (task >> 2) / SEGS;
        const int64_t e = cb * kStep + 32 * g + 8 * (task & 3);
        const bool ok = task < TASKS && e < A.K;
        const float * xp = A.x + (ok ? n * A.x_s1 + e : 0);
        const float4 u = *reinterpret_cast<const float4 *>(xp);
        const float4 w = *reinterpret_cast<const float4 *>(xp + 4);
        xe[p][0] = ok ? u.x : 0.0f; xe[p][1] = ok ? u.y : 0.0f; xe[p][2] = ok ? u.z : 0.0f; xe[p][3] = ok ? u.w : 0.0f;
        xe[p][4] = ok ? w.x : 0.0f; xe[p][5] = ok ? w.y : 0.0f; xe[p][6] = ok ? w.z : 0.0f; xe[p][7] = ok ? w.w : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);
    const int j = rt >= A.tstart[1] ? (rt >= A.tstart[2] ? 2 : 1) : 0;
    const int64_t M = A.M[j], m0 = (rt - A.tstart[j]) * R, mw = m0 + 32 * rw;
    F f;
    {
        const int64_t m = min(mw + r, M - 1), g0 = m & ~(int64_t) 31;
        f.init(A.w[j], M, A.nb, g0, (int) min<int64_t>(32, M - g0), (int) (m - g0), h);
    }
    Raw buf[SPW];
    // (step 0's weights before the x conversion, step 1's after it, as in k_mvb)
    buf[0] = f.load(ns > 0 ? sb : 0);
    __builtin_amdgcn_sched_barrier(0);

    XSeg * xs = reinterpret_cast<XSeg *>(lds);                                  // [NC][SEGS]
    float4 * xf = reinterpret_cast<float4 *>(xs + NC * SEGS);                   // [NC][SEGS]
    float * red = reinterpret_cast<float *>(xf + NC * SEGS);                    // [KW][RW][NC][32]
    uint8_t * zpad = reinterpret_cast<uint8_t *>(red + KW * RW * NC * 32);
    if (tid < 4) reinterpret_cast<uint32_t *>(zpad)[tid] = 0u;
    bool sp = false;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int task = p * T + tid, g = (task >> 2) % SEGS, n = task < TASKS ? (task >> 2) / SEGS : 0;
        // (tasks past the last column convert zeros into a segment index past SEGS: not stored)
        sp |= convert_seg(xe[p], task < TASKS ? g : SEGS, SEGS, task & 3, xs + n * SEGS, xf + n * SEGS);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 1; s < SPW; ++s) buf[s] = f.load(s < ns ? sb + s : (ns > 0 ? sb : 0));
    __builtin_amdgcn_sched_barrier(0);
    const bool special = __syncthreads_or(sp); // (also: x and zpad are in LDS for every wave)

    // the lane's A operand: row i = 4 blk + k (plane k < 3), k-half h
    const int blk = r >> 2, k = r & 3;
    int acol = -1; // the column of set 0 (set s adds s * CPS), -1: zeros
    if (k < 3) {
        if constexpr (DT == Q6_K) acol = ((blk & 1) == h) ? (blk >> 1) : -1;
        else acol = blk;
    }
    const int aoff = k * 32 + h * 16;
    float acc[NS][4];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[s][i] = 0.0f;
#pragma unroll
    for (int st = 0; st < SPW; ++st) {
        if (st < ns) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int sg = (kw * SPW + st) * kSegs + F::seg(q);
                const v4i B = f.bop(buf[st], q);
                const float2 fc = f.fac(buf[st], q);
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    const int n = acol + s * CPS;
                    const uint8_t * pa = (acol >= 0 && n < NC) ? reinterpret_cast<const uint8_t *>(xs + n * SEGS + sg) + aoff : zpad;
                    const v16i D = mfma32(*reinterpret_cast<const v4i *>(pa), B);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        // D rows 8 i + 4 h + (0..2): column 2 i + h (Q6_K: i, group h) of the set
                        const int col = s * CPS + (DT == Q6_K ? i : 2 * i + h);
                        if (col < NC) {
                            const float4 xfv = xf[col * SEGS + sg];
                            const float P = planes(D[4 * i], D[4 * i + 1], D[4 * i + 2]);
                            if constexpr (F::OFF) acc[s][i] = fmaf(fc.x * xfv.x, P, fmaf(fc.y, xfv.w, acc[s][i]));
                            else acc[s][i] = fmaf(fc.x * xfv.x, P, acc[s][i]);
                        }
                    }
                }
            }
        }
    }
    // this wave's sums per (column, row)
    float * rw_red = red + (kw * RW + rw) * NC * 32;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = acc[s][i];
            if constexpr (DT == Q6_K) v += __shfl_xor(v, 32); // the row's two 16-element groups
            const int col = s * CPS + (DT == Q6_K ? i : 2 * i + h);
            if (col < NC && (DT != Q6_K || h == 0)) rw_red[col * 32 + r] = v;
        }
    }
    // the exact sums of flagged x segments of the wave's steps (no accumulator live any more)
    if (special) {
        for (int n = 0; n < NC; ++n) {
            const float * xn = A.x + n * A.x_s1;
            uint64_t fm = 0;
            for (int g = 0; g < ns * kSegs; ++g) fm |= (uint64_t) flagged_at(xf + n * SEGS, kw * SPW * kSegs + g) << g;
            if (fm != 0) {
                exact_red_n<DT>(A.w[j], M, A.nb, mw, xn, fm, 1, ns * kSegs, sb * kStep, rw_red + n * 32);
                exact_red_n<DT>(A.w[j], M, A.nb, mw + 16, xn, fm, 1, ns * kSegs, sb * kStep, rw_red + n * 32 + 16);
            }
        }
    }
    __syncthreads();
    // the K waves' sums in order, then y or the chunk's partial sums
    for (int t = tid; t < NC * R; t += T) {
        const int n = t / R, rr = t % R;
        float v = 0.0f;
#pragma unroll
        for (int k2 = 0; k2 < KW; ++k2) v += red[((k2 * RW + rr / 32) * NC + n) * 32 + rr % 32];
        if (A.nchunks == 1) {
            if (m0 + rr < M) A.y[j][n * A.ys1[j] + m0 + rr] = v;
        } else {
            // agent-scope stores (written through the XCD's L2), waited for below
            __hip_atomic_store(A.part + ((int64_t) c * NC + n) * A.prow + rt * R + rr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (A.nchunks == 1) return;
    __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): this wave's partial-sum stores are done
    __syncthreads();
    // the count moves after every storing wave's write-through stores are acknowledged (the
    // ordering of k_mvc); the last chunk of the tile adds all of them in chunk order and puts the
    // count back to zero
    uint32_t & last = *reinterpret_cast<uint32_t *>(zpad + 16);
    if (tid == 0) last = __hip_atomic_fetch_add(A.arrive + rt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t) A.nchunks - 1;
    __syncthreads();
    if (!last) return;
    for (int t = tid; t < NC * R; t += T) {
        const int n = t / R, rr = t % R;
        if (m0 + rr < M) {
            A.y[j][n * A.ys1[j] + m0 + rr] = ordered_sum(A.part + n * A.prow + rt * R + rr, NC * A.prow, A.nchunks);
        }
    }
    if (tid == 0) __hip_atomic_store(A.arrive + rt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// waves per work-group: row waves x K waves (measured on the config shapes at N = 2, 4, 8 against
// 2 x 4, 1 x 8, 2 x 8, 2 x 2, 2 x 1 and 8 x 1: 4 x 2 the fastest or within 5% everywhere)
constexpr int kMwRW = 4, kMwKW = 2;
// K of 32 steps or more (down projections: few rows, long K): 2 row waves x 4 K waves, K chunks
// of 8 steps (half the chunks to hand over). Measured against 4 x 2 (one box): Q8_0 4096 x 11008
// at N = 2 / 4 / 8 15.2 / 15.2 / 18.0 -> 14.0 / 14.2 / 17.0 us, Q4_K 4096 x 12288 at N = 8 14.9 ->
// 14.6, Q6_K 4096 x 12288 at N = 4 even; at 16 steps it lost (the Q6_K LM head at N = 8 148 -> 163,
// gate+up 20.3-20.7 -> 21.4 us)
int tuning(const char * name, int dflt);

struct MwShape {
    int rw, kw;
};
inline MwShape mw_shape(int64_t nst) {
    static const bool on = tuning("SCRAPGPU_HIP_MV_MW_LONG", 1) != 0;
    return on && nst >= 32 ? MwShape{2, 4} : MwShape{kMwRW, kMwKW};
}

template <int DT, int RW, int KW>
void * pick_mvw_s(int nc) {
    switch (nc) {
        case 2: return (void *) k_mvw<DT, 2, RW, KW>;
        case 3: return (void *) k_mvw<DT, 3, RW, KW>;
        case 4: return (void *) k_mvw<DT, 4, RW, KW>;
        case 5: return (void *) k_mvw<DT, 5, RW, KW>;
        case 6: return (void *) k_mvw<DT, 6, RW, KW>;
        case 7: return (void *) k_mvw<DT, 7, RW, KW>;
        default: return (void *) k_mvw<DT, 8, RW, KW>;
    }
}

template <int DT>
void * pick_mvw(int nc, MwShape sh) {
    return sh.rw == 2 ? pick_mvw_s<DT, 2, 4>(nc) : pick_mvw_s<DT, kMwRW, kMwKW>(nc);
}

template <int DT, bool PRE>
void * pick_mvc_p(int nc) {
    switch (nc) {
        case 2: return (void *) k_mvc<DT, 2, PRE>;
        case 3: return (void *) k_mvc<DT, 3, PRE>;
        case 4: return (void *) k_mvc<DT, 4, PRE>;
        case 5: return (void *) k_mvc<DT, 5, PRE>;
        case 6: return (void *) k_mvc<DT, 6, PRE>;
        case 7: return (void *) k_mvc<DT, 7, PRE>;
        default: return (void *) k_mvc<DT, 8, PRE>;
    }
}

template <int DT>
void * pick_mvc(int nc, bool pre) {
    return pre ? pick_mvc_p<DT, true>(nc) : pick_mvc_p<DT, false>(nc);
}

template <int DT, int RG>
void * pick_burst_rg(int W, int spw) {
    // the instances a launch can ask for: 2-step waves in any even count up to 16 (and 2, 4); on
    // 16-row tiles also 4-step waves (3..12 of them, Q8_0 excepted past 8) and 3-step waves (Q8_0:
    // 11..16; the other formats: 16) -- the launcher picks W and spw
    if (spw <= 2) {
        switch (W) {
            case 2: return (void *) k_mvb<DT, RG, 2, 2>;
            case 4: return (void *) k_mvb<DT, RG, 4, 2>;
            case 6: return (void *) k_mvb<DT, RG, 6, 2>;
            case 8: return (void *) k_mvb<DT, RG, 8, 2>;
            case 10: return (void *) k_mvb<DT, RG, 10, 2>;
            case 12: return (void *) k_mvb<DT, RG, 12, 2>;
            case 14: return (void *) k_mvb<DT, RG, 14, 2>;
            default: return (void *) k_mvb<DT, RG, 16, 2>;
        }
    }
    if constexpr (RG == 1) {
        if (spw == 3) {
            if constexpr (DT == Q8_0) {
                switch (W) {
                    case 11: return (void *) k_mvb<DT, 1, 11, 3>;
                    case 12: return (void *) k_mvb<DT, 1, 12, 3>;
                    case 13: return (void *) k_mvb<DT, 1, 13, 3>;
                    case 14: return (void *) k_mvb<DT, 1, 14, 3>;
                    case 15: return (void *) k_mvb<DT, 1, 15, 3>;
                    default: break;
                }
            }
            return (void *) k_mvb<DT, 1, 16, 3>;
        }
        switch (W) {
            case 3: return (void *) k_mvb<DT, 1, 3, 4>;
            case 5: return (void *) k_mvb<DT, 1, 5, 4>;
            case 6: return (void *) k_mvb<DT, 1, 6, 4>;
            case 7: return (void *) k_mvb<DT, 1, 7, 4>;
            default: break;
        }
        if constexpr (DT != Q8_0) {
            switch (W) {
                case 9: return (void *) k_mvb<DT, 1, 9, 4>;
                case 10: return (void *) k_mvb<DT, 1, 10, 4>;
                case 11: return (void *) k_mvb<DT, 1, 11, 4>;
                case 12: return (void *) k_mvb<DT, 1, 12, 4>;
                default: break;
            }
        }
    }
    return W >= 16 ? (void *) k_mvb<DT, RG, 16, 4> : W >= 8 ? (void *) k_mvb<DT, RG, 8, 4> : (void *) k_mvb<DT, RG, 4, 4>;
}

template <int DT>
void * pick_burst(int W, int spw, int rg) {
    return rg == 3 ? pick_burst_rg<DT, 3>(W, spw) : rg == 2 ? pick_burst_rg<DT, 2>(W, spw) : pick_burst_rg<DT, 1>(W, spw);
}

// MUL_MAT_ID pairs with K of up to 32 steps: the instances that issue the expert id's load with
// the x loads (others read it through where_of, one round trip ahead of them)
template <int DT, int RG>
void * pick_burst_id_rg(int W) {
    return W >= 16 ? (void *) k_mvb<DT, RG, 16, 2, false, true> : W >= 8 ? (void *) k_mvb<DT, RG, 8, 2, false, true>
         : W >= 4 ? (void *) k_mvb<DT, RG, 4, 2, false, true> : (void *) k_mvb<DT, RG, 2, 2, false, true>;
}

template <int DT>
void * pick_burst_id(int W, int rg) {
    return rg == 3 ? pick_burst_id_rg<DT, 3>(W) : rg == 2 ? pick_burst_id_rg<DT, 2>(W) : pick_burst_id_rg<DT, 1>(W);
}

// streaming variants: W = 8 for one column, 4 for several
template <int DT>
void * pick_stream(int nc) {
    switch (nc) {
        case 1: return (void *) k_mvs<DT, 1, 8>;
        case 2: return (void *) k_mvs<DT, 2, 4>;
        case 3: return (void *) k_mvs<DT, 3, 4>;
        case 4: return (void *) k_mvs<DT, 4, 4>;
        case 5: return (void *) k_mvs<DT, 5, 4>;
        case 6: return (void *) k_mvs<DT, 6, 4>;
        case 7: return (void *) k_mvs<DT, 7, 4>;
        default: return (void *) k_mvs<DT, 8, 4>;
    }
}

// resident work-groups per CU of a kernel at a block size and dynamic LDS (cached per thread)
int occupancy(void * fn, int threads, size_t lds) {
    struct Key {
        void * fn;
        size_t lds;
        int n;
    };
    thread_local std::vector<Key> cache;
    for (const Key & k : cache)
        if (k.fn == fn && k.lds == lds) return k.n;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, lds) != hipSuccess || n < 1) n = 1;
    cache.push_back({fn, lds, n});
    return n;
}

// tuning overrides from the environment (0 / unset = automatic)
int tuning(const char * name, int dflt) {
    const char * v = std::getenv(name);
    return v != nullptr && *v ? std::atoi(v) : dflt;
}

const char * name_of(int dt, int nmat) {
    if (nmat > 1) {
        switch (dt) {
            case Q4_0: return "matvec_multi_q4_0";
            case Q8_0: return "matvec_multi_q8_0";
            case Q4_K: return "matvec_multi_q4_k";
            default: return "matvec_multi_q6_k";
        }
    }
    switch (dt) {
        case Q4_0: return "matvec_q4_0";
        case Q8_0: return "matvec_q8_0";
        case Q4_K: return "matvec_q4_k";
        default: return "matvec_q6_k";
    }
}

void set_tiles(MvArgs & L, const MatArgs * mats, int nmat, int R) {
    L.tstart[0] = 0;
    for (int j = 0; j < 3; ++j) L.tstart[j + 1] = j < nmat ? L.tstart[j] + (mats[j].M + R - 1) / R : INT64_MAX;
    L.tiles = L.tstart[nmat];
}

} // namespace

// the multi-column form applies (several columns, one slice, not MUL_MAT_ID)
static bool mc_form(const MatArgs * mats, int nmat, const IdArgs * id) {
    static const bool on = [] {
        const char * v = std::getenv("SCRAPGPU_HIP_MV_MC");
        return v == nullptr || v[0] != '0';
    }();
    (void) nmat;
    return on && id == nullptr && mats[0].N >= 2 && mats[0].N <= 8 && mats[0].ne12 * mats[0].ne13 == 1;
}

// the chunked burst applies (one column, one slice, not MUL_MAT_ID, K of 17..64 steps, at most
// kArriveMax 16-row tiles); it also needs x 16-byte aligned, checked at launch
static bool chunk_form(const MatArgs * mats, int nmat, const IdArgs * id) {
    static const bool on = [] {
        const char * v = std::getenv("SCRAPGPU_HIP_MV_CHUNK");
        return v == nullptr || v[0] != '0';
    }();
    if (!on || id != nullptr || mats[0].N != 1) return false;
    const int64_t nst = (mats[0].K + kStep - 1) / kStep;
    int64_t tiles = 0;
    for (int j = 0; j < nmat; ++j) {
        if (mats[j].ne12 * mats[j].ne13 != 1) return false;
        tiles += (mats[j].M + 15) / 16;
    }
    return nst > kChunkSteps && nst <= 64 && tiles <= kArriveMax;
}

static size_t chunk_part_bytes(const MatArgs * mats, int nmat) {
    const int64_t nst = (mats[0].K + kStep - 1) / kStep, nck = (nst + kChunkSteps - 1) / kChunkSteps;
    int64_t tiles = 0;
    // (rows of each matrix rounded up to its 16-, 32- or 48-row tiles: at most 32 past 16-row ones)
    for (int j = 0; j < nmat; ++j) tiles += (mats[j].M + 15) / 16 + 2;
    return ((size_t) nck * (size_t) tiles * 16 * sizeof(float) + 255) / 256 * 256;
}

size_t matvec_scratch_bytes(const MatArgs * mats, int nmat, const IdArgs * id) {
    if (nmat >= 1 && is_float_weight(mats[0].dtype)) return 0;
    if (nmat >= 1 && chunk_form(mats, nmat, id)) return chunk_part_bytes(mats, nmat);
    if (nmat < 1 || !mc_form(mats, nmat, id)) return 0;
    const int64_t nst = (mats[0].K + kStep - 1) / kStep, nchunks = (nst + kMcChunk - 1) / kMcChunk, nsegp = nchunks * kMcChunk * kSegs;
    int64_t tiles = 0, rows_w = 0;
    const MwShape mws = mw_shape(nst);
    for (int j = 0; j < nmat; ++j) {
        tiles += (mats[j].M + 15) / 16;
        rows_w += (mats[j].M + 32 * mws.rw - 1) / (32 * mws.rw) * (32 * mws.rw);
    }
    const size_t nc = (size_t) mats[0].N;
    // k_mvc: x planes and factors, K-chunk partial sums and counts
    size_t b = (nc * (size_t) nsegp * sizeof(XSeg) + 255) / 256 * 256 + (nc * (size_t) nsegp * sizeof(float4) + 255) / 256 * 256;
    if (nchunks > 1) b += ((size_t) nchunks * nc * (size_t) tiles * 16 * sizeof(float) + 255) / 256 * 256 + (size_t) tiles * sizeof(uint32_t);
    // k_mvw: K-chunk partial sums
    const int64_t wchunks = (nst + 2 * mws.kw - 1) / (2 * mws.kw);
    const size_t bw = wchunks > 1 ? ((size_t) wchunks * nc * (size_t) rows_w * sizeof(float) + 255) / 256 * 256 : 0;
    return std::max<size_t>(std::max<size_t>(b, bw), 256);
}

hipError_t launch_matvec(const MatArgs * mats, int nmat, int cu_count, hipStream_t stream, const char ** kernel_name,
                         uint64_t * grid_size, const IdArgs * id, uint8_t * scratch, uint32_t * arrive) {
    if (nmat < 1 || nmat > 3) return hipErrorInvalidValue;
    const MatArgs & a = mats[0];
    if (is_float_weight(a.dtype)) return launch_matvec_float(mats, nmat, stream, kernel_name, grid_size, id);
    for (int j = 0; j < nmat; ++j) {
        if (mats[j].dtype != a.dtype || mats[j].K != a.K || mats[j].N != a.N || (nmat > 1 && mats[j].ne12 * mats[j].ne13 != 1)) {
            return hipErrorInvalidValue;
        }
    }
    const int nc = (int) a.N;
    if (nc < 1 || nc > 8 || a.K <= 0 || a.K % 32 != 0) return hipErrorInvalidValue;
    if (id != nullptr && (nc != 1 || id->ids == nullptr || id->n_used < 1 || id->n_tok < 1 || id->n_exp < 1)) return hipErrorInvalidValue;
    for (int j = 1; j < nmat && id != nullptr; ++j) {
        // several expert tensors under one ids: one expert stride and one output layout
        if (mats[j].w_s2 != a.w_s2 || mats[j].y_s1 != a.y_s1 || mats[j].y_s2 != a.y_s2) return hipErrorInvalidValue;
    }
    const int64_t slices = id != nullptr ? id->n_used * id->n_tok : a.ne12 * a.ne13;
    if (slices < 1 || slices > 65535) return hipErrorInvalidValue;
    const int dt = a.dtype;
    if (dt != Q4_0 && dt != Q8_0 && dt != Q4_K && dt != Q6_K) return hipErrorInvalidValue;
    int64_t rows = 0;
    for (int j = 0; j < nmat; ++j) rows += mats[j].M;
    if ((rows + 15) / 16 > 0x7FFFFFFF) return hipErrorInvalidValue;

    MvArgs L;
    for (int j = 0; j < 3; ++j) {
        const bool has = j < nmat;
        L.w[j] = has ? mats[j].w : nullptr;
        L.M[j] = has ? mats[j].M : 0;
        L.y[j] = has ? mats[j].y : nullptr;
        L.ys1[j] = has ? mats[j].y_s1 : 0;
    }
    const int64_t nst = (a.K + kStep - 1) / kStep;
    L.K = a.K;
    L.nb = a.K / (dt == Q4_K || dt == Q6_K ? 256 : 32);
    L.nst = nst;
    L.x = a.x;
    L.x_s1 = a.x_s1;
    L.x_s2 = a.x_s2;
    L.x_s3 = a.x_s3;
    L.w_s2 = a.w_s2;
    L.w_s3 = a.w_s3;
    L.y_s2 = a.y_s2;
    L.y_s3 = a.y_s3;
    L.ne12 = a.ne12;
    L.r2 = a.r2;
    L.r3 = a.r3;
    L.xvec = ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && (a.x_s1 & 3) == 0 && (a.x_s2 & 3) == 0 && (a.x_s3 & 3) == 0) ? 1 : 0;
    L.ids = id != nullptr ? id->ids : nullptr;
    L.ids_s0 = id != nullptr ? id->s0 : 0;
    L.ids_s1 = id != nullptr ? id->s1 : 0;
    L.n_used = id != nullptr ? id->n_used : 1;
    L.n_exp = id != nullptr ? id->n_exp : 1;
    L.x_shared = id != nullptr ? id->x_shared : 0;
    if (kernel_name) *kernel_name = name_of(dt, nmat);

    // burst form (one column, K <= 64 steps): every wave's steps (<= 4) loaded at once, one tile
    // per work-group. 32- or 48-row tiles (two or three row groups sharing each x operand) for
    // large products, 16-row tiles otherwise (more work-groups). 2 steps per wave up to K = 32 steps, 3 up to 48 (16 waves), then 4.
    L.nck = 1;
    L.part = nullptr;
    L.arrive = nullptr;
    if (nc == 1 && L.xvec && scratch != nullptr && arrive != nullptr && chunk_form(mats, nmat, id) &&
        rows >= (int64_t) tuning("SCRAPGPU_HIP_MV_CHUNK_ROWS", 64) * cu_count &&
        tuning("SCRAPGPU_HIP_MV_BURST", 1)) {
        // a long K in chunks of kChunkSteps steps over 8-wave work-groups of 16 rows, once there
        // are 4 row tiles per CU: the chunks' hand-over (partial-sum stores, the arrival count,
        // the last chunk's loads) adds dependent memory round trips at the end of the launch,
        // which cost more than smaller work-groups save below that (Q6_K 4096 x 12288: 11.8
        // against 10.7 us; Q4_K 28672 x 8192: 30.7 against 32.1 us)
        // (Q4 products: 48-row tiles, three row groups sharing each x operand, from 96 rows per CU)
        const bool q4 = dt == Q4_K || dt == Q4_0;
        int rg = q4 && rows >= (int64_t) 96 * cu_count ? 3 : 1;
        if (const int fr = tuning("SCRAPGPU_HIP_MV_CHUNK_RG", 0)) rg = q4 && fr >= 3 ? 3 : q4 && fr == 2 ? 2 : 1;
        set_tiles(L, mats, nmat, 16 * rg);
        L.nck = (nst + kChunkSteps - 1) / kChunkSteps;
        L.part = reinterpret_cast<float *>(scratch);
        L.arrive = arrive;
        constexpr int W = 8, sp = 2;
        const size_t lds = (size_t) W * sp * kSegs * (sizeof(XSeg) + sizeof(float4)) + (size_t) W * 16 * rg * sizeof(float) + 32;
        void * fn = dt == Q8_0 ? (void *) k_mvb<Q8_0, 1, W, sp, true> : dt == Q6_K ? (void *) k_mvb<Q6_K, 1, W, sp, true>
                  : dt == Q4_0 ? (rg == 3 ? (void *) k_mvb<Q4_0, 3, W, sp, true> : rg == 2 ? (void *) k_mvb<Q4_0, 2, W, sp, true> : (void *) k_mvb<Q4_0, 1, W, sp, true>)
                               : (rg == 3 ? (void *) k_mvb<Q4_K, 3, W, sp, true> : rg == 2 ? (void *) k_mvb<Q4_K, 2, W, sp, true> : (void *) k_mvb<Q4_K, 1, W, sp, true>);
        const uint64_t grid = (uint64_t) L.tiles * (uint64_t) L.nck;
        if (grid_size) *grid_size = grid;
        std::snprintf(last_form().form, sizeof(last_form().form), "burst-chunks rg=%d W=%d spw=%d chunks=%d", rg, W, sp, (int) L.nck);
        last_form().grid = grid;
        void * args[] = {&L};
        return hipLaunchKernel(fn, dim3((unsigned) L.tiles, (unsigned) L.nck), dim3((unsigned) (64 * W)), args, lds, stream);
    }
    if (nc == 1 && L.xvec && nst <= 64 && tuning("SCRAPGPU_HIP_MV_BURST", 1)) {
        // (the 32-row Q8_0 / Q6_K forms need more registers than 5 waves per SIMD leave them)
        // 48-row tiles once they give every CU two work-groups (one round at 4 waves per SIMD),
        // 32-row ones from 24 rows per CU (with the non-temporal weight loads the Q4_K q/k/v
        // launch, 6144 rows, 5.06 against 5.28 us on 16-row tiles; o at 4096 rows stays on 16)
        const bool q4 = dt == Q4_K || dt == Q4_0;
        // (past 32 steps of K, 16-row tiles: the 32- and 48-row forms spill at 3-4 steps per wave)
        int rg = q4 && rows * slices >= (int64_t) 96 * cu_count ? 3 : q4 && rows * slices >= (int64_t) tuning("SCRAPGPU_HIP_MV_RG2_ROWS", 24) * cu_count ? 2 : 1;
        // MUL_MAT_ID pairs: 16-row tiles (the Qwen3-30B-A3B MoE token's Q4_K gate+up pairs, 8 x
        // 1536 rows: 32-row tiles 0.480 ms per 48-layer token, 16-row ones 0.474-0.475; A/B on one box)
        if (L.ids != nullptr && tuning("SCRAPGPU_HIP_MV_ID_RG1", 1)) rg = 1;
        if (const int fr = tuning("SCRAPGPU_HIP_MV_RG", 0)) rg = fr >= 3 ? 3 : fr >= 2 ? 2 : 1;
        if (nst > 32) rg = 1; // (also over the override)
        // 3 steps per wave for 33..48 steps on 16 waves (below: as many waves as K needs)
        int sp = nst <= 32 ? 2 : nst <= 48 && rg == 1 && tuning("SCRAPGPU_HIP_MV_SPW3", 1) ? 3 : 4;
        // (K of 4 steps or fewer: 2 waves, so that none is left without a step: the MoE experts'
        // Q6_K down projection, K = 768, as 1024 2-wave work-groups: a 4-layer MoE token
        // 53.7-55.2 -> 49.5-50.2 us)
        int W = nst <= 2 * sp ? 2 : 4;
        while (W < 16 && (nst + W - 1) / W > sp) W *= 2;
        // 2 steps per wave: an even number of waves, the fewest that cover K (at most 3 loads
        // unused: 20 steps as 10 waves, not 16 with 12 of them reloading a step), whose count need
        // not be a power of two. Against the power of two on one box: Q4_K 5120 x 5120 (20
        // steps) 8.4-8.5 -> 6.6 us, 13824 x 5120 13.4 -> 11.2, Q8_0 5120 x 5120 11.1 -> 8.5,
        // Q6_K 10.3 -> 8.3, Q4_K 4096 x 6144 (24 steps) 5.8 -> 5.2, 8192 x 7168 (28 steps) 8.6 ->
        // 8.5. (MUL_MAT_ID pairs keep the power of two: the instances that read the id ahead.)
        if (sp == 2 && nst > 8 && L.ids == nullptr && tuning("SCRAPGPU_HIP_MV_W2", 1)) W = (int) std::min<int64_t>(16, 2 * ((nst + 3) / 4));
        // Q4_0 / Q4_K / Q6_K with 33..48 steps: ceil(steps / 4) waves of 4 steps (9..12 waves, at most
        // 3 loads unused), against 16 waves of 3: the Q6_K down projection (48 steps) 9.9 -> 9.5-9.6
        // us and the token 1.074 -> 1.064 ms; 44-step Q4_0 8.4-8.5 -> 7.7, 40-step Q4_K 8.1-8.3 ->
        // 7.25, 38-step Q6_K 9.9 -> 9.0 us. Q8_0 (its larger step registers: 4 steps measured 11.1-11.2
        // -> 11.3-11.4 us on 4096 x 11008) takes ceil(steps / 3) waves of 3 steps: 4096 x 11008 (43
        // steps, 15 waves) 11.15-11.22 -> 10.8, 4096 x 10240 (40 steps, 14 waves) 11.3 -> 10.7 us
        // 16-row tiles at 16 or more per CU (the LM head's 9496): 4-step waves, ceil(steps / 4) of
        // them, against 2-step ones (A/B on two boxes): Q6_K 151936 x 4096 87.6 -> 84.1-85.0 and
        // 93.9-95.7 -> 90.7-92.9 us, Q8_0 108 -> 105; at 4 tiles per CU (16384 rows) 11.8 -> 12.6-12.9,
        // at 8 (32000 rows) 20.3-21.1 -> 21.2-21.3, at one (4096 x 4096) 3.98 -> 5.07, and on 32- and
        // 48-row tiles (they spill) it loses
        if (sp == 2 && rg == 1 && nst > 8 && L.ids == nullptr && rows * slices >= (int64_t) 256 * cu_count && tuning("SCRAPGPU_HIP_MV_S4", 1)) {
            sp = 4;
            W = (int) ((nst + 3) / 4);
        }
        if (nst > 32 && nst <= 48 && rg == 1 && tuning("SCRAPGPU_HIP_MV_W4", 1)) {
            sp = dt == Q8_0 ? 3 : 4;
            W = (int) ((nst + sp - 1) / sp);
        }
        set_tiles(L, mats, nmat, 16 * rg);
        L.cs = sp;
        const size_t lds = (size_t) W * sp * kSegs * (sizeof(XSeg) + sizeof(float4)) + (size_t) W * 16 * rg * sizeof(float) + 16;
        static const bool id_early = tuning("SCRAPGPU_HIP_MV_ID_EARLY", 1) != 0;
        void * fn = dt == Q4_0 ? pick_burst<Q4_0>(W, sp, rg) : dt == Q8_0 ? pick_burst<Q8_0>(W, sp, rg)
                  : dt == Q4_K ? pick_burst<Q4_K>(W, sp, rg) : pick_burst<Q6_K>(W, sp, rg);
        if (L.ids != nullptr && sp == 2 && id_early)
            fn = dt == Q4_0 ? pick_burst_id<Q4_0>(W, rg) : dt == Q8_0 ? pick_burst_id<Q8_0>(W, rg)
               : dt == Q4_K ? pick_burst_id<Q4_K>(W, rg) : pick_burst_id<Q6_K>(W, rg);
        if (grid_size) *grid_size = (uint64_t) L.tiles * (uint64_t) slices;
        std::snprintf(last_form().form, sizeof(last_form().form), "burst rg=%d W=%d spw=%d", rg, W, sp);
        last_form().grid = (uint64_t) L.tiles * (uint64_t) slices;
        void * args[] = {&L};
        return hipLaunchKernel(fn, dim3((unsigned) L.tiles, (unsigned) slices), dim3((unsigned) (64 * W)), args, lds, stream);
    }

    // several columns, one slice: k_mvw (128-row tiles x K chunks of 4 steps on 32x32x32 MFMAs, x
    // converted in the kernel), which needs x 16-byte aligned and the stream's arrival counts; else
    // (or SCRAPGPU_HIP_MV_MW=0) k_mvc
    static const bool mw_on = tuning("SCRAPGPU_HIP_MV_MW", 1) != 0;
    if (mw_on && scratch != nullptr && arrive != nullptr && L.xvec && mc_form(mats, nmat, id)) {
        const MwShape mws = mw_shape(nst);
        const int R = 32 * mws.rw, CH = 2 * mws.kw;
        MwArgs C;
        std::memset(&C, 0, sizeof(C));
        for (int j = 0; j < 3; ++j) {
            const bool has = j < nmat;
            C.w[j] = has ? mats[j].w : nullptr;
            C.M[j] = has ? mats[j].M : 0;
            C.y[j] = has ? mats[j].y : nullptr;
            C.ys1[j] = has ? mats[j].y_s1 : 0;
            C.tstart[j + 1] = has ? C.tstart[j] + (mats[j].M + R - 1) / R : INT64_MAX;
        }
        const int64_t tiles = C.tstart[nmat];
        if (tiles > kArriveMax) return hipErrorInvalidValue;
        C.nb = L.nb;
        C.nst = nst;
        C.K = a.K;
        C.nchunks = (nst + CH - 1) / CH;
        C.x = a.x;
        C.x_s1 = a.x_s1;
        C.part = reinterpret_cast<float *>(scratch);
        C.arrive = arrive;
        C.prow = tiles * R;
        void * fn = dt == Q4_0 ? pick_mvw<Q4_0>(nc, mws) : dt == Q8_0 ? pick_mvw<Q8_0>(nc, mws) : dt == Q4_K ? pick_mvw<Q4_K>(nc, mws) : pick_mvw<Q6_K>(nc, mws);
        const size_t lds = (size_t) nc * CH * kSegs * (sizeof(XSeg) + sizeof(float4)) + (size_t) mws.kw * mws.rw * nc * 32 * sizeof(float) + 32;
        if (lds > 65536) {
            static std::mutex mu;
            std::lock_guard<std::mutex> lock(mu);
            const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
            if (e != hipSuccess) return e;
        }
        if (grid_size) *grid_size = (uint64_t) tiles * (uint64_t) C.nchunks;
        std::snprintf(last_form().form, sizeof(last_form().form), "columns mfma32 nc=%d chunks=%d", nc, (int) C.nchunks);
        last_form().grid = (uint64_t) tiles * (uint64_t) C.nchunks;
        void * args[] = {&C};
        return hipLaunchKernel(fn, dim3((unsigned) tiles, (unsigned) C.nchunks), dim3(64 * mws.rw * mws.kw), args, lds, stream);
    }
    if (scratch != nullptr && mc_form(mats, nmat, id)) {
        // several columns: x pre-pass, then one work-group per 16 rows and K chunk
        McArgs C;
        std::memset(&C, 0, sizeof(C));
        C.tstart[0] = 0;
        for (int j = 0; j < 3; ++j) {
            const bool has = j < nmat;
            C.w[j] = has ? mats[j].w : nullptr;
            C.M[j] = has ? mats[j].M : 0;
            C.y[j] = has ? mats[j].y : nullptr;
            C.ys1[j] = has ? mats[j].y_s1 : 0;
            C.tstart[j + 1] = has ? C.tstart[j] + (mats[j].M + 15) / 16 : INT64_MAX;
        }
        const int64_t tiles = C.tstart[nmat];
        C.nb = L.nb;
        C.nst = nst;
        C.nchunks = (nst + kMcChunk - 1) / kMcChunk;
        C.nsegp = C.nchunks * kMcChunk * kSegs;
        XSeg * planes = reinterpret_cast<XSeg *>(scratch);
        float4 * fac = reinterpret_cast<float4 *>(scratch + ((size_t) nc * C.nsegp * sizeof(XSeg) + 255) / 256 * 256);
        C.planes = planes;
        C.fac = fac;
        C.prow = tiles * 16;
        C.part = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(fac) + ((size_t) nc * C.nsegp * sizeof(float4) + 255) / 256 * 256);
        C.arrive = reinterpret_cast<uint32_t *>(reinterpret_cast<uint8_t *>(C.part) + ((size_t) C.nchunks * nc * (size_t) C.prow * sizeof(float) + 255) / 256 * 256);
        C.x = a.x;
        C.x_s1 = a.x_s1;
        C.K = a.K;
        // the x pre-pass once the columns are many (SCRAPGPU_HIP_MV_PRE: the smallest column count
        // that takes it; x must be 16-byte aligned for the in-kernel conversion)
        static const int pre_from = tuning("SCRAPGPU_HIP_MV_PRE", 4);
        // (several K chunks: the pre-pass also clears their arrival counters)
        const bool pre = nc >= pre_from || !L.xvec || C.nchunks > 1;
        hipError_t e = hipSuccess;
        if (pre) {
            hipLaunchKernelGGL(k_x_planes, dim3((unsigned) (C.nsegp / 16), (unsigned) nc), dim3(64), 0, stream, a.x, a.x_s1, a.K, C.nsegp, planes, fac,
                               C.arrive, C.nchunks > 1 ? tiles : (int64_t) 0);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        void * fn = dt == Q4_0 ? pick_mvc<Q4_0>(nc, pre) : dt == Q8_0 ? pick_mvc<Q8_0>(nc, pre) : dt == Q4_K ? pick_mvc<Q4_K>(nc, pre) : pick_mvc<Q6_K>(nc, pre);
        const size_t lds = (size_t) kMcW * std::min(nc, 4) * kMcSpw * kSegs * (sizeof(XSeg) + sizeof(float4)) + (size_t) kMcW * nc * 16 * sizeof(float) + 32;
        if (lds > 65536) {
            static std::mutex mu;
            std::lock_guard<std::mutex> lock(mu);
            if ((e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds)) != hipSuccess) return e;
        }
        if (grid_size) *grid_size = (uint64_t) tiles * (uint64_t) C.nchunks;
        std::snprintf(last_form().form, sizeof(last_form().form), "columns nc=%d chunks=%d%s", nc, (int) C.nchunks, pre ? " pre" : "");
        last_form().grid = (uint64_t) tiles * (uint64_t) C.nchunks;
        void * args[] = {&C};
        return hipLaunchKernel(fn, dim3((unsigned) tiles, (unsigned) C.nchunks), dim3(64 * kMcW), args, lds, stream);
    }

    // streaming form (several columns, or K too long for the burst form)
    set_tiles(L, mats, nmat, 16);
    const int W = nc == 1 ? 8 : 4;
    // x chunk per wave: all of the wave's steps when they fit the LDS budget, else as many as fit
    const int64_t step_bytes = (int64_t) kSegs * nc * (sizeof(XSeg) + sizeof(float4));
    const int64_t per_wave = std::max<int64_t>(1, (nst + W - 1) / W);
    const int64_t cs = std::min<int64_t>(per_wave, std::max<int64_t>(1, kLdsX / W / step_bytes));
    L.cs = (int) cs;
    const size_t lds = (size_t) W * cs * step_bytes + (size_t) 2 * W * nc * 16 * sizeof(float) + 16;
    if (lds > (size_t) 160 * 1024) return hipErrorInvalidValue;
    // several columns: the columns share each MFMA (k_mvn); SCRAPGPU_HIP_MV_COLS=0 runs one MFMA
    // set per column (k_mvs)
    void * fn = nullptr;
    if (nc >= 2 && tuning("SCRAPGPU_HIP_MV_COLS", 1)) {
        fn = dt == Q4_0 ? pick_columns<Q4_0>(nc) : dt == Q8_0 ? pick_columns<Q8_0>(nc) : dt == Q4_K ? pick_columns<Q4_K>(nc) : pick_columns<Q6_K>(nc);
    } else {
        fn = dt == Q4_0 ? pick_stream<Q4_0>(nc) : dt == Q8_0 ? pick_stream<Q8_0>(nc) : dt == Q4_K ? pick_stream<Q4_K>(nc) : pick_stream<Q6_K>(nc);
    }

    // persistent grid: as many work-groups as stay resident (at most one per tile), trimmed so
    // that every work-group gets the same number of tiles
    const int per_cu = std::max(1, tuning("SCRAPGPU_HIP_MV_WGS", occupancy(fn, 64 * W, lds)));
    const int64_t cap = std::max<int64_t>(1, (int64_t) per_cu * cu_count / slices);
    const int64_t rounds = (L.tiles + cap - 1) / cap;
    const int64_t grid_x = (L.tiles + rounds - 1) / rounds;
    if (grid_size) *grid_size = (uint64_t) grid_x * (uint64_t) slices;
    std::snprintf(last_form().form, sizeof(last_form().form), "%s nc=%d W=%d", nc >= 2 && tuning("SCRAPGPU_HIP_MV_COLS", 1) ? "stream-columns" : "stream", nc, W);
    last_form().grid = (uint64_t) grid_x * (uint64_t) slices;
    void * args[] = {&L};
    return hipLaunchKernel(fn, dim3((unsigned) grid_x, (unsigned) slices), dim3((unsigned) (64 * W)), args, lds, stream);
}

} // namespace sgk
