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
// column, so the 16 rows of A are used to keep apart what must be scaled separately: row 4c + k
// of A holds, for k-group c only, plane k % 2 of x over the scale group that lane group c needs
// (k / 2 selects one of two scale groups), and zeros elsewhere. After the 4 MFMAs of a step, lane
// (r, p) finds in its 4 accumulator registers (rows 4p .. 4p + 3 of D, column r) exactly the 2 x 2
// integer sums its part needs, and applies the block scales once per scale group. Per 64 weights a
// lane spends ~30 VALU operations (unpack + scales) instead of ~110 with VALU dot products, which
// leaves the VALU idle enough to overlap the HBM stream.
//
// x conversion. Every 32-element segment of x is stored as two int8 planes a, b and a scale s
// (s = max|x| / 127): x ~= s * a + (s / 253) * b, plus the plain sums of its two 16-element
// halves:
//   sum_i q_i x_i ~= (s / 253) * (253 * sum q a + sum q b)
// with each format's constant offset applied once per scale group through the segment sums:
//   Q4_0: d * (sum q x - 8 sum x)            Q8_0: d * sum q x      (q = stored byte xor 0x80)
//   Q4_K: d*sc * sum q x - dmin*m * sum x    Q6_K: d*sc * (sum q x - 32 sum x)
// The two planes carry ~15 significant bits of each x relative to its segment's largest |x|, so
// the product differs from the fp32 reference by ~1e-5 of max|x| per term, well inside the
// NMSE <= 1e-7 bound of the decode path.
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
};

__device__ __forceinline__ float half_bits(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short) (h & 0xFFFFu)));
}

__device__ __forceinline__ uint4 load16(const uint8_t * p) {
    return *reinterpret_cast<const uint4 *>(p);
}

__device__ __forceinline__ uint32_t load_half(const uint8_t * p) {
    return *reinterpret_cast<const uint16_t *>(p);
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

// 253 * (sum over plane a) + (sum over plane b), as float
__device__ __forceinline__ float planes(int da, int db) {
    return (float) (da * 253 + db);
}

// one x segment in LDS: plane a (32 int8), plane b (32 int8)
struct XSeg {
    uint4 a0, a1, b0, b1;
};

// The converted x of one wave's chunk, per column n: xs[n * nseg + g] (planes) and
// xf[n * nseg + g] = {s / 253, sum of elements 0..15, sum of elements 16..31, sum of all 32}.
// zpad: 16 zero bytes, the A operand of lanes that carry no x.
struct XView {
    const XSeg * xs;
    const float4 * xf;
    const uint8_t * zpad;
    int nseg;
};

// ---- per format ----------------------------------------------------------------------------------
// init() resolves the lane's row in every R32 area once (Q4_K, Q8_0, Q4_0: as 32-bit byte offsets
// from the matrix slice's base w, which is uniform across the work-group and so stays in scalar
// registers; a slice is < 4 GiB, checked on the host); load(step) fetches what the lane needs of
// one step, branch-free; bop(raw, t) is the lane's B operand (16 int8 codes) for MFMA t = 0..3 of the step;
// aoff(t, c, k, g) is the byte offset, inside the step's XSeg run, of the 16 x bytes that lane
// (row 4c + k of A, k-group g) supplies to MFMA t, or -1 for zeros; flush() scales the integer
// sums of lane part p into the row sum.

template <int DT> struct Fmt;

// Q4_K: a step is one block; part p takes chunk p (64 elements: units 2p, 2p + 1 of the 128
// nibble bytes): sub-block 2p (low nibbles), 2p + 1 (high). MFMA t takes elements 64p + 16t .. +15
// (t = 0, 1: low nibbles of units 2p, 2p + 1; t = 2, 3: high nibbles). A row 4c + k: plane k % 2
// of sub-block 2c + k / 2.
template <>
struct Fmt<Q4_K> {
    static constexpr int ND = 1; // accumulator sets per step
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
        if (c != g || (k >> 1) != (t >> 1)) return -1;
        return (2 * g + (t >> 1)) * 64 + (k & 1) * 32 + (t & 1) * 16;
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
        float a = (d * sc0) * f0.x * planes(D[0].x, D[0].y);
        a = fmaf(-dmin * m0, f0.w, a);
        a = fmaf((d * sc1) * f1.x, planes(D[0].z, D[0].w), a);
        return fmaf(-dmin * m1, f1.w, a);
    }
};

// Q6_K: a step is one block; part p takes task p = (h, hf): the 64 elements 128h + 32t + 16hf + i
// (t, i < 4, 16) built from ql units 4h + hf, 4h + 2 + hf and qh unit 8 + 2h + hf; MFMA t takes
// the 16 of run t, which has its own signed 8-bit scale. Two accumulator sets (t = 0, 1 and
// t = 2, 3); A row 4c + k of set u: plane k % 2 of run 2u + k / 2 of task c.
template <>
struct Fmt<Q6_K> {
    static constexpr int ND = 2;
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
        if (c != g || (k >> 1) != (t & 1)) return -1;
        const int h = g >> 1, hf = g & 1;
        return (4 * h + t) * 64 + (k & 1) * 32 + hf * 16;
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
            const v4i & Dt = D[t >> 1];
            const int ia = (t & 1) ? Dt.z : Dt.x, ib = (t & 1) ? Dt.w : Dt.y;
            const float4 f = xf[4 * h + t];
            const float s16 = hf ? f.z : f.y;
            a = fmaf(ds, fmaf(f.x, planes(ia, ib), -32.0f * s16), a);
        }
        return a;
    }
};

// Q8_0: a step is 8 blocks of 32; MFMA t takes blocks 2t, 2t + 1 (part p: half p % 2 of block
// 2t + p / 2); part p scales blocks 2p, 2p + 1. A row 4c + k: plane k % 2 of block 2c + k / 2.
// Blocks past the end of the row (K % 256 != 0) load block 0 and contribute with d = 0.
template <>
struct Fmt<Q8_0> {
    static constexpr int ND = 1;
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
        const uint32_t b0 = (uint32_t) step * 8 + 2 * p, b1 = b0 + 1;
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
        if (c != t || (k >> 1) != (g >> 1)) return -1;
        return (2 * t + (g >> 1)) * 64 + (k & 1) * 32 + (g & 1) * 16;
    }
    __device__ float flush(const Raw & r, const v4i * D, const float4 * xf) const {
        const float a = half_bits(r.d0) * xf[2 * p].x * planes(D[0].x, D[0].y);
        return fmaf(half_bits(r.d1) * xf[2 * p + 1].x, planes(D[0].z, D[0].w), a);
    }
};

// Q4_0: a step is 8 blocks of 32 (16 nibble bytes each: low nibbles = elements 0..15, high =
// 16..31); part p takes blocks p and p + 4. MFMA t: blocks 0..3 (t < 2) or 4..7, half t % 2.
// A row 4c + k: plane k % 2 of block c + 4 (k / 2).
template <>
struct Fmt<Q4_0> {
    static constexpr int ND = 1;
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
        if (c != g || (k >> 1) != (t >> 1)) return -1;
        return (g + 4 * (t >> 1)) * 64 + (k & 1) * 32 + (t & 1) * 16;
    }
    __device__ float flush(const Raw & r, const v4i * D, const float4 * xf) const {
        const float4 fa = xf[p], fb = xf[p + 4];
        const float a = half_bits(r.da) * fmaf(fa.x, planes(D[0].x, D[0].y), -8.0f * fa.w);
        return fmaf(half_bits(r.db), fmaf(fb.x, planes(D[0].z, D[0].w), -8.0f * fb.w), a);
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
                const int u = ND == 1 ? 0 : (t >> 1);
                D[u] = mfma(Aop[t], Fmt<DT>::bop(raw[i], t), D[u]);
            }
            acc[i][n] += f[i].flush(raw[i], D, xf);
        }
    }
}

// ---- x conversion ----------------------------------------------------------------------------------

// Segment g (of nseg) of a wave's range, elements 8q .. 8q + 7 held by this lane in v (lanes
// 4k .. 4k + 3 hold one segment): two int8 planes, the plane scale and the plain sums. Rounding
// to integers: adding 1.5 * 2^23 leaves the nearest integer in the low mantissa bits.
__device__ __forceinline__ void convert_seg(const float (&v)[8], int g, int nseg, int q, XSeg * xs, float4 * xf) {
    constexpr float kMagic = 12582912.0f; // 1.5 * 2^23
    float amax = 0.0f, sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        amax = fmaxf(amax, fabsf(v[i]));
        sum += v[i];
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const float s16 = sum + __shfl_xor(sum, 1);
    const float s32 = s16 + __shfl_xor(s16, 2);
    const float s16o = __shfl_xor(s16, 2);
    const float sc = amax * (1.0f / 127.0f);
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    const float invb = 253.0f * inv;
    uint32_t pa[2], pb[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint32_t ba[4], bb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float t = v[4 * h + i];
            const float fa = fmaf(t, inv, kMagic);                          // |a| <= 127
            const float fb = fmaf(fmaf(kMagic - fa, sc, t), invb, kMagic); // |b| <= 127 (253 < 254)
            ba[i] = __float_as_uint(fa);
            bb[i] = __float_as_uint(fb);
        }
        // byte i of the result = byte 0 of word i
        pa[h] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(ba[3], ba[2], 0x0c0c0400u), __builtin_amdgcn_perm(ba[1], ba[0], 0x0c0c0400u),
                                      0x05040100u);
        pb[h] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(bb[3], bb[2], 0x0c0c0400u), __builtin_amdgcn_perm(bb[1], bb[0], 0x0c0c0400u),
                                      0x05040100u);
    }
    if (g < nseg) {
        uint8_t * sp = reinterpret_cast<uint8_t *>(xs + g);
        *reinterpret_cast<uint2 *>(sp + 8 * q) = make_uint2(pa[0], pa[1]);
        *reinterpret_cast<uint2 *>(sp + 32 + 8 * q) = make_uint2(pb[0], pb[1]);
        if (q == 0) xf[g] = make_float4(sc * (1.0f / 253.0f), s16, s16o, s32);
    }
}

// The wave's chunk of nseg segments starting at element e0, for NC columns. Lane l converts
// elements 8 (l % 4) .. +8 of segment l / 4 (16 segments per pass); elements past K are zero.
template <int NC>
__device__ void convert_x(const MvArgs & A, const float * x, int64_t e0, int nseg, int lane, XSeg * xs, float4 * xf) {
    const int q = lane & 3;
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
            convert_seg(v, g, nseg, q, xs + n * nseg, xf + n * nseg);
        }
    }
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
template <int RG, int NC, int W>
__device__ __forceinline__ void reduce_store(const MvArgs & A, const Where & wh, const Row & row, float (&acc)[RG][NC], float * red, int tid) {
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

// Burst form (one column, <= SPW steps per wave, one tile of 16 * RG rows per work-group): the wave
// first loads its x range, then issues every weight load, and only then converts x.
template <int DT, int RG, int W, int SPW>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(SPW <= 2 && RG == 1 ? 6 : SPW <= 2 && RG == 2 ? 5 : 4, 8))) void k_mvb(MvArgs A) {
    using F = Fmt<DT>;
    using Raw = typename F::Raw;
    extern __shared__ uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const Where wh = where_of(A);

    const int64_t s0 = A.nst * wave / W, s1 = A.nst * (wave + 1) / W;
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
    F f[RG];
    const Row row = row_of<DT, RG>(A, blockIdx.x, wh.w_off, lane & 15, lane >> 4, f);
    Raw buf[SPW][RG];
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
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
#pragma unroll
    for (int p = 0; p < XP; ++p) convert_seg(xv[p], 16 * p + (lane >> 2), nseg, lane & 3, xs, xf);
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
    reduce_store<RG, 1, W>(A, wh, row, acc, red, tid);
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
    if (once && ns > 0) convert_x<NC>(A, wh.x, s0 * kStep, ns * kSegs, lane, xs, xf);
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
                convert_x<NC>(A, wh.x, (s0 + k) * kStep, min(cs, ns - k) * kSegs, lane, xs, xf);
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
            cur[0] = nxt[0];
        }
        reduce_store<1, NC, W>(A, wh, row, acc, red + (it & 1) * (W * NC * 16), tid);
        tile = ntile;
        row = nrow;
        f[0] = fn[0];
    }
}

template <int DT, int RG>
void * pick_burst_rg(int W, int spw) {
    if (spw <= 2) return W >= 16 ? (void *) k_mvb<DT, RG, 16, 2> : W >= 8 ? (void *) k_mvb<DT, RG, 8, 2> : (void *) k_mvb<DT, RG, 4, 2>;
    if constexpr (RG == 1) {
        if (spw == 3) return (void *) k_mvb<DT, 1, 16, 3>; // (W = 16 only; 16-row tiles only)
    }
    return W >= 16 ? (void *) k_mvb<DT, RG, 16, 4> : W >= 8 ? (void *) k_mvb<DT, RG, 8, 4> : (void *) k_mvb<DT, RG, 4, 4>;
}

template <int DT>
void * pick_burst(int W, int spw, int rg) {
    return rg == 3 ? pick_burst_rg<DT, 3>(W, spw) : rg == 2 ? pick_burst_rg<DT, 2>(W, spw) : pick_burst_rg<DT, 1>(W, spw);
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

hipError_t launch_matvec(const MatArgs * mats, int nmat, int cu_count, hipStream_t stream, const char ** kernel_name,
                         uint64_t * grid_size, const IdArgs * id) {
    if (nmat < 1 || nmat > 3) return hipErrorInvalidValue;
    const MatArgs & a = mats[0];
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
    if (nc == 1 && L.xvec && nst <= 64 && tuning("SCRAPGPU_HIP_MV_BURST", 1)) {
        // (the 32-row Q8_0 / Q6_K forms need more registers than 5 waves per SIMD leave them)
        // 48-row tiles once they give every CU two work-groups (one round at 4 waves per SIMD)
        const bool q4 = dt == Q4_K || dt == Q4_0;
        // (past 32 steps of K, 16-row tiles: the 32- and 48-row forms spill at 3-4 steps per wave)
        int rg = q4 && rows * slices >= (int64_t) 96 * cu_count ? 3 : q4 && rows * slices >= (int64_t) 64 * cu_count ? 2 : 1;
        if (const int fr = tuning("SCRAPGPU_HIP_MV_RG", 0)) rg = fr >= 3 ? 3 : fr >= 2 ? 2 : 1;
        if (nst > 32) rg = 1; // (also over the override)
        // 3 steps per wave for 33..48 steps (16 waves: no wave loads a step it does not use)
        const int sp = nst <= 32 ? 2 : nst <= 48 && rg == 1 && tuning("SCRAPGPU_HIP_MV_SPW3", 1) ? 3 : 4;
        int W = 4;
        while (W < 16 && (nst + W - 1) / W > sp) W *= 2;
        set_tiles(L, mats, nmat, 16 * rg);
        L.cs = sp;
        const size_t lds = (size_t) W * sp * kSegs * (sizeof(XSeg) + sizeof(float4)) + (size_t) W * 16 * rg * sizeof(float) + 16;
        void * fn = dt == Q4_0 ? pick_burst<Q4_0>(W, sp, rg) : dt == Q8_0 ? pick_burst<Q8_0>(W, sp, rg)
                  : dt == Q4_K ? pick_burst<Q4_K>(W, sp, rg) : pick_burst<Q6_K>(W, sp, rg);
        if (grid_size) *grid_size = (uint64_t) L.tiles * (uint64_t) slices;
        std::snprintf(last_form().form, sizeof(last_form().form), "burst rg=%d W=%d spw=%d", rg, W, sp);
        last_form().grid = (uint64_t) L.tiles * (uint64_t) slices;
        void * args[] = {&L};
        return hipLaunchKernel(fn, dim3((unsigned) L.tiles, (unsigned) slices), dim3((unsigned) (64 * W)), args, lds, stream);
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
    void * fn = dt == Q4_0 ? pick_stream<Q4_0>(nc) : dt == Q8_0 ? pick_stream<Q8_0>(nc) : dt == Q4_K ? pick_stream<Q4_K>(nc) : pick_stream<Q6_K>(nc);

    // persistent grid: as many work-groups as stay resident (at most one per tile), trimmed so
    // that every work-group gets the same number of tiles
    const int per_cu = std::max(1, tuning("SCRAPGPU_HIP_MV_WGS", occupancy(fn, 64 * W, lds)));
    const int64_t cap = std::max<int64_t>(1, (int64_t) per_cu * cu_count / slices);
    const int64_t rounds = (L.tiles + cap - 1) / cap;
    const int64_t grid_x = (L.tiles + rounds - 1) / rounds;
    if (grid_size) *grid_size = (uint64_t) grid_x * (uint64_t) slices;
    std::snprintf(last_form().form, sizeof(last_form().form), "stream nc=%d W=%d", nc, W);
    last_form().grid = (uint64_t) grid_x * (uint64_t) slices;
    void * args[] = {&L};
    return hipLaunchKernel(fn, dim3((unsigned) grid_x, (unsigned) slices), dim3((unsigned) (64 * W)), args, lds, stream);
}

} // namespace sgk
