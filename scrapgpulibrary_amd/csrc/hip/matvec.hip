// Decode matvec over R32 weights for 1 <= N <= 8 columns (gfx950, wave64).
//
// Replaces, for the hip backend, the reference's R32 matvec kernels k_mvr_* / k_mvrc_*
// (src/backends/opencl11/kernels/mul_mv_r.cl:240-287), k_mvr_q4_k / k_mvr_q6_k (mul_mv_k.cl:396-450)
// and, for 2-3 weights sharing x, k_mvm_* (mul_mv_multi.cl:46-99). Same products, new design.
//
// Work decomposition. A work-group owns a tile of R rows (R = 16 or 32, inside one R32 group of
// 32 rows) and all of K. Its W waves split K into contiguous ranges of steps (a step = 256
// elements), so a wave only needs its own part of x, which it converts into its private LDS
// region; the waves meet once, at the end, to add their partial row sums in a fixed order.
//
// Inside a wave, lane l serves row r = l % R through part p = l / R (P = 64 / R parts). A step's
// bytes of one row are dealt to the parts by whole scale groups, so one 128-bit wave load reads P
// runs of 16 * R contiguous bytes of one R32 unit area (256 B or 512 B): coalesced.
//
// Two forms:
//  * burst (N = 1, K <= 64 steps): one tile per work-group, at most 4 steps per wave; the wave
//    loads its x range, then issues every weight load, and only then converts x, so the x round
//    trip hides under the weight round trip. No loop-carried state: few registers, 4-8 waves per
//    SIMD, and the hardware dispatcher streams the work-groups.
//  * streaming (N > 1, or longer K): a persistent grid; each work-group walks tiles, its waves
//    convert their x range once (when it fits the LDS budget) and keep the next step's loads in
//    flight while computing the current one.
//
// x conversion. Every 32-element segment of x is stored as two int8 planes a, b and a scale s
// (s = max|x| / 127): x ~= s * a + (s / 253) * b, plus the plain sums of its two 16-element
// halves. A weight run then costs one sdot4 per 4 weights and plane:
//   sum_i q_i x_i ~= (s / 253) * (253 * sum q a + sum q b)
// with block scales factored out and each format's constant offset applied once per run through
// the segment sums:
//   Q4_0: d * (sum q x - 8 sum x)            Q8_0: d * sum q x      (q = stored byte xor 0x80)
//   Q4_K: d*sc * sum q x - dmin*m * sum x    Q6_K: d*sc * (sum q x - 32 sum x)
// The two planes carry ~15 significant bits of each x relative to its segment's largest |x|, so
// the product differs from the fp32 reference by ~1e-5 of max|x| per term, well inside the
// NMSE <= 1e-7 bound of the decode path.
#include "kernels.h"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <vector>

namespace sgk {
namespace {

constexpr int kStep = 256;     // K elements per step
constexpr int kSegs = 8;       // 32-element x segments per step
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
    int cs;   // steps per x chunk of one wave
    int64_t tiles; // row tiles over all matrices
    int xvec; // x columns are 16-byte aligned: float4 loads
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

// one x segment in LDS: a plane (32 int8), b plane (32 int8)
struct XSeg {
    uint4 a0, a1, b0, b1;
};

// 253 * (q . a) + (q . b) over 16 int8 pairs (four words of q against 16 bytes of each plane)
__device__ __forceinline__ int dot16(uint4 q, uint4 a, uint4 b) {
    int ta = __builtin_amdgcn_sdot4((int) q.x, (int) a.x, 0, false);
    ta = __builtin_amdgcn_sdot4((int) q.y, (int) a.y, ta, false);
    ta = __builtin_amdgcn_sdot4((int) q.z, (int) a.z, ta, false);
    ta = __builtin_amdgcn_sdot4((int) q.w, (int) a.w, ta, false);
    int tb = __builtin_amdgcn_sdot4((int) q.x, (int) b.x, 0, false);
    tb = __builtin_amdgcn_sdot4((int) q.y, (int) b.y, tb, false);
    tb = __builtin_amdgcn_sdot4((int) q.z, (int) b.z, tb, false);
    tb = __builtin_amdgcn_sdot4((int) q.w, (int) b.w, tb, false);
    return ta * 253 + tb;
}

// the same over 32 pairs: q0 against the first 16 bytes of the segment, q1 against the last 16
__device__ __forceinline__ int dot32(uint4 q0, uint4 q1, const XSeg & s) {
    int ta = __builtin_amdgcn_sdot4((int) q0.x, (int) s.a0.x, 0, false);
    ta = __builtin_amdgcn_sdot4((int) q0.y, (int) s.a0.y, ta, false);
    ta = __builtin_amdgcn_sdot4((int) q0.z, (int) s.a0.z, ta, false);
    ta = __builtin_amdgcn_sdot4((int) q0.w, (int) s.a0.w, ta, false);
    ta = __builtin_amdgcn_sdot4((int) q1.x, (int) s.a1.x, ta, false);
    ta = __builtin_amdgcn_sdot4((int) q1.y, (int) s.a1.y, ta, false);
    ta = __builtin_amdgcn_sdot4((int) q1.z, (int) s.a1.z, ta, false);
    ta = __builtin_amdgcn_sdot4((int) q1.w, (int) s.a1.w, ta, false);
    int tb = __builtin_amdgcn_sdot4((int) q0.x, (int) s.b0.x, 0, false);
    tb = __builtin_amdgcn_sdot4((int) q0.y, (int) s.b0.y, tb, false);
    tb = __builtin_amdgcn_sdot4((int) q0.z, (int) s.b0.z, tb, false);
    tb = __builtin_amdgcn_sdot4((int) q0.w, (int) s.b0.w, tb, false);
    tb = __builtin_amdgcn_sdot4((int) q1.x, (int) s.b1.x, tb, false);
    tb = __builtin_amdgcn_sdot4((int) q1.y, (int) s.b1.y, tb, false);
    tb = __builtin_amdgcn_sdot4((int) q1.z, (int) s.b1.z, tb, false);
    tb = __builtin_amdgcn_sdot4((int) q1.w, (int) s.b1.w, tb, false);
    return ta * 253 + tb;
}

__device__ __forceinline__ uint4 lo4(uint4 q) {
    return make_uint4(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu);
}
__device__ __forceinline__ uint4 hi4(uint4 q) {
    return make_uint4((q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu, (q.z >> 4) & 0x0F0F0F0Fu, (q.w >> 4) & 0x0F0F0F0Fu);
}

// The converted x of one wave's chunk: xs[n * nseg + g] (planes) and xf[n * nseg + g] =
// {s / 253, sum of elements 0..15, sum of elements 16..31, sum of all 32}.
struct XView {
    const XSeg * xs;
    const float4 * xf;
    int nseg;
};

// ---- per format: the lane's slice of a step ------------------------------------------------------
// init() resolves the lane's row in every R32 area once; load(step) fetches what the lane needs of
// one step; compute() accumulates it for NC columns against x segments of the current chunk
// (sg0 = index of the step's first segment inside the chunk).

template <int DT, int R> struct Fmt;

// Q4_K: a step is one block; part p takes chunks c = p, p + P, ... (64 elements: 32 bytes = units
// 2c, 2c + 1 of the 128 nibble bytes), i.e. whole sub-blocks 2c (low nibbles), 2c + 1 (high).
template <int R>
struct Fmt<Q4_K, R> {
    static constexpr int P = 64 / R;
    static constexpr int CL = 4 / P; // chunks per lane
    struct Raw {
        uint4 q[CL][2];
        uint4 hd;
    };
    const uint8_t * qb;
    const uint8_t * hb;
    uint32_t qblk, qunit, hblk;
    int p;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb, int64_t g0, int rs, int lr, int part, int64_t) {
        p = part;
        qb = w + (uint64_t) g0 * nb * 128 + (uint64_t) lr * 16;
        hb = w + (uint64_t) M * nb * 128 + (uint64_t) g0 * nb * 16 + (uint64_t) lr * 16;
        qblk = (uint32_t) rs * 128;
        qunit = (uint32_t) rs * 16;
        hblk = (uint32_t) rs * 16;
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        const uint8_t * b = qb + (uint32_t) step * qblk;
#pragma unroll
        for (int i = 0; i < CL; ++i) {
            const int c = p + P * i;
            r.q[i][0] = load16(b + (uint32_t) (2 * c) * qunit);
            r.q[i][1] = load16(b + (uint32_t) (2 * c + 1) * qunit);
        }
        r.hd = load16(hb + (uint32_t) step * hblk);
        return r;
    }
    template <int NC>
    __device__ void compute(const Raw & r, int sg0, const XView & xv, float * acc) const {
        const float d = half_bits(r.hd.x), dmin = half_bits(r.hd.x >> 16);
        const uint32_t s0 = r.hd.y, s1 = r.hd.z, s2 = r.hd.w; // scale bytes 0..3, 4..7, 8..11
#pragma unroll
        for (int i = 0; i < CL; ++i) {
            const int c = p + P * i;
            // sub-blocks 2c (low nibbles) and 2c + 1 (high nibbles): 6-bit scale and min
            float sc0, m0, sc1, m1;
            const int sh0 = 16 * (c & 1), sh1 = sh0 + 8; // byte (2c) & 3, (2c + 1) & 3
            if (c < 2) {
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
            const float d0 = d * sc0, d1 = d * sc1, n0 = -dmin * m0, n1 = -dmin * m1;
            const uint4 l0 = lo4(r.q[i][0]), l1 = lo4(r.q[i][1]);
            const uint4 h0 = hi4(r.q[i][0]), h1 = hi4(r.q[i][1]);
            const int g = sg0 + 2 * c;
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                const int gi = n * xv.nseg + g;
                const float4 f0 = xv.xf[gi], f1 = xv.xf[gi + 1];
                float a = acc[n];
                a = fmaf(d0 * f0.x, (float) dot32(l0, l1, xv.xs[gi]), a);
                a = fmaf(n0, f0.w, a);
                a = fmaf(d1 * f1.x, (float) dot32(h0, h1, xv.xs[gi + 1]), a);
                a = fmaf(n1, f1.w, a);
                acc[n] = a;
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
};

// Q6_K: a step is one block; part p takes tasks k = p, p + P, ... (h = k >> 1, hf = k & 1): the
// 64 elements 128h + 32rr + 16hf + i (rr, i < 4, 16) built from ql units 4h + hf, 4h + 2 + hf and
// qh unit 8 + 2h + hf; each 16-run has its own signed 8-bit scale.
template <int R>
struct Fmt<Q6_K, R> {
    static constexpr int P = 64 / R;
    static constexpr int TL = 4 / P; // tasks per lane
    struct Raw {
        uint4 qa[TL], qc[TL], qh[TL];
        uint4 sc;
        uint32_t d;
    };
    const uint8_t * qb;
    const uint8_t * sb;
    const uint8_t * db;
    uint32_t qblk, qunit, sblk, dblk;
    int p;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb, int64_t g0, int rs, int lr, int part, int64_t) {
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
        const uint8_t * b = qb + (uint32_t) step * qblk;
#pragma unroll
        for (int t = 0; t < TL; ++t) {
            const int k = p + P * t, h = k >> 1, hf = k & 1;
            r.qa[t] = load16(b + (uint32_t) (4 * h + hf) * qunit);
            r.qc[t] = load16(b + (uint32_t) (4 * h + 2 + hf) * qunit);
            r.qh[t] = load16(b + (uint32_t) (8 + 2 * h + hf) * qunit);
        }
        r.sc = load16(sb + (uint32_t) step * sblk);
        r.d = load_half(db + (uint32_t) step * dblk);
        return r;
    }
    template <int NC>
    __device__ void compute(const Raw & r, int sg0, const XView & xv, float * acc) const {
        const float d = half_bits(r.d);
#pragma unroll
        for (int t = 0; t < TL; ++t) {
            const int k = p + P * t, h = k >> 1, hf = k & 1;
            const uint4 qa = r.qa[t], qc = r.qc[t], qh = r.qh[t];
            // scale of run rr: byte 8h + hf + 2rr of the 16 (stored xor 0x80, so value = byte - 128)
            const uint32_t sw0 = h ? r.sc.z : r.sc.x, sw1 = h ? r.sc.w : r.sc.y;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                // 6-bit values of run rr: low nibbles of qa (rr 0) / qc (rr 1), high nibbles (rr 2, 3),
                // with bits 2rr, 2rr + 1 of qh on top
                const uint4 ql = (rr & 1) ? qc : qa;
                const int ls = rr < 2 ? 0 : 4;
                const int hs = 2 * rr;
                const uint4 v = make_uint4(((ql.x >> ls) & 0x0F0F0F0Fu) | (((qh.x >> hs) << 4) & 0x30303030u),
                                           ((ql.y >> ls) & 0x0F0F0F0Fu) | (((qh.y >> hs) << 4) & 0x30303030u),
                                           ((ql.z >> ls) & 0x0F0F0F0Fu) | (((qh.z >> hs) << 4) & 0x30303030u),
                                           ((ql.w >> ls) & 0x0F0F0F0Fu) | (((qh.w >> hs) << 4) & 0x30303030u));
                const uint32_t sw = rr < 2 ? sw0 : sw1;
                const int bi = 2 * (rr & 1) + hf;
                const float ds = d * ((float) ((sw >> (8 * bi)) & 0xFFu) - 128.0f);
                const int g = sg0 + 4 * h + rr;
#pragma unroll
                for (int n = 0; n < NC; ++n) {
                    const int gi = n * xv.nseg + g;
                    // this lane's 16-element half of the segment: planes and plain sum
                    const uint4 * pl = reinterpret_cast<const uint4 *>(xv.xs + gi) + hf;
                    const float * fp = reinterpret_cast<const float *>(xv.xf + gi);
                    const int tq = dot16(v, pl[0], pl[2]);
                    const float sum16 = fp[1 + hf];
                    const float4 f = make_float4(fp[0], 0.0f, 0.0f, 0.0f);
                    acc[n] = fmaf(ds, fmaf(f.x, (float) tq, -32.0f * sum16), acc[n]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }
};

// Q8_0 / Q4_0: a step is 8 blocks of 32; part p takes blocks p, p + P, ... of the step. Blocks past
// the end of the row (K % 256 != 0) load block 0 and contribute with d = 0.
template <int R>
struct Fmt<Q8_0, R> {
    static constexpr int P = 64 / R;
    static constexpr int BL = 8 / P; // blocks per lane and step
    struct Raw {
        uint4 q[BL][2];
        uint32_t d[BL];
    };
    const uint8_t * qb;
    const uint8_t * db;
    uint32_t qblk, qunit, dblk;
    int64_t nb;
    int p;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb_, int64_t g0, int rs, int lr, int part, int64_t) {
        p = part;
        nb = nb_;
        qb = w + (uint64_t) g0 * nb * 32 + (uint64_t) lr * 16;
        db = w + (uint64_t) M * nb * 32 + (uint64_t) g0 * nb * 2 + (uint64_t) lr * 2;
        qblk = (uint32_t) rs * 32;
        qunit = (uint32_t) rs * 16;
        dblk = (uint32_t) rs * 2;
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            int64_t b = step * 8 + p + P * i;
            const bool ok = b < nb;
            b = ok ? b : 0;
            r.q[i][0] = load16(qb + (uint32_t) b * qblk);
            r.q[i][1] = load16(qb + (uint32_t) b * qblk + qunit);
            r.d[i] = ok ? load_half(db + (uint32_t) b * dblk) : 0u;
        }
        return r;
    }
    template <int NC>
    __device__ void compute(const Raw & r, int sg0, const XView & xv, float * acc) const {
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            const float d = half_bits(r.d[i]);
            const uint4 a = r.q[i][0], b = r.q[i][1];
            const uint4 q0 = make_uint4(a.x ^ 0x80808080u, a.y ^ 0x80808080u, a.z ^ 0x80808080u, a.w ^ 0x80808080u);
            const uint4 q1 = make_uint4(b.x ^ 0x80808080u, b.y ^ 0x80808080u, b.z ^ 0x80808080u, b.w ^ 0x80808080u);
            const int g = sg0 + p + P * i;
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                const int gi = n * xv.nseg + g;
                acc[n] = fmaf(d * xv.xf[gi].x, (float) dot32(q0, q1, xv.xs[gi]), acc[n]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
};

template <int R>
struct Fmt<Q4_0, R> {
    static constexpr int P = 64 / R;
    static constexpr int BL = 8 / P;
    struct Raw {
        uint4 q[BL];
        uint32_t d[BL];
    };
    const uint8_t * qb;
    const uint8_t * db;
    uint32_t qblk, dblk;
    int64_t nb;
    int p;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb_, int64_t g0, int rs, int lr, int part, int64_t) {
        p = part;
        nb = nb_;
        qb = w + (uint64_t) g0 * nb * 16 + (uint64_t) lr * 16;
        db = w + (uint64_t) M * nb * 16 + (uint64_t) g0 * nb * 2 + (uint64_t) lr * 2;
        qblk = (uint32_t) rs * 16;
        dblk = (uint32_t) rs * 2;
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            int64_t b = step * 8 + p + P * i;
            const bool ok = b < nb;
            b = ok ? b : 0;
            r.q[i] = load16(qb + (uint32_t) b * qblk);
            r.d[i] = ok ? load_half(db + (uint32_t) b * dblk) : 0u;
        }
        return r;
    }
    template <int NC>
    __device__ void compute(const Raw & r, int sg0, const XView & xv, float * acc) const {
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            const float d = half_bits(r.d[i]);
            const uint4 l = lo4(r.q[i]), h = hi4(r.q[i]); // elements 0..15, 16..31 of the block
            const int g = sg0 + p + P * i;
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                const int gi = n * xv.nseg + g;
                const float4 f = xv.xf[gi];
                const int t = dot32(l, h, xv.xs[gi]);
                acc[n] = fmaf(d, fmaf(f.x, (float) t, -8.0f * f.w), acc[n]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
};

// ---- x conversion of one wave's chunk --------------------------------------------------------------
// Lane l converts elements 8 (l % 4) .. +8 of segment l / 4 (16 segments per pass of the wave);
// elements past K are zero.
// Segment g (of nseg) of a wave's range, elements 8q .. 8q + 7 held by this lane in v (lanes
// 4k .. 4k + 3 hold one segment): two int8 planes, the plane scale and the plain sums.
__device__ __forceinline__ void convert_seg(const float (&v)[8], int g, int nseg, int q, XSeg * xs, float4 * xf) {
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
        uint32_t wa = 0, wb = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float t = v[4 * h + i];
            const float qa = rintf(t * inv);                 // |qa| <= 127
            const float qb = rintf(fmaf(-qa, sc, t) * invb); // |qb| <= 127 (253 < 254 leaves headroom)
            wa |= ((uint32_t) (int) qa & 0xFFu) << (8 * i);
            wb |= ((uint32_t) (int) qb & 0xFFu) << (8 * i);
        }
        pa[h] = wa;
        pb[h] = wb;
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

// Burst form for short wave ranges (<= SPW steps per wave, one column, one tile per work-group):
// the wave first loads its x range, then issues every weight load, and only then converts x, so
// the x round trip overlaps the weight round trip and a work-group costs about one HBM latency.
template <int DT, int R, int W, int SPW>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_mvb(MvArgs A) {
    using F = Fmt<DT, R>;
    using Raw = typename F::Raw;
    extern __shared__ uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane % R, part = lane / R;

    const int64_t sl = blockIdx.y;
    const int64_t i2 = sl % A.ne12, i3 = sl / A.ne12;
    const uint64_t w_off = (uint64_t) (i2 / A.r2) * A.w_s2 + (uint64_t) (i3 / A.r3) * A.w_s3;
    const float * x = A.x + i2 * A.x_s2 + i3 * A.x_s3;

    const int64_t tile = blockIdx.x;
    const int j = tile >= A.tstart[1] ? (tile >= A.tstart[2] ? 2 : 1) : 0;
    const int64_t M = A.M[j];
    const int64_t m0 = (tile - A.tstart[j]) * R;
    const int64_t g0 = m0 & ~(int64_t) 31;
    const int rs = (int) min<int64_t>(32, M - g0);
    const int lr = m0 + r < M ? (int) (m0 - g0) + r : rs - 1; // dead lanes read a real row and drop it

    const int64_t s0 = A.nst * wave / W, s1 = A.nst * (wave + 1) / W;
    const int ns = (int) (s1 - s0);

    // x: lane l holds elements 8 (l % 4) .. +8 of segment l / 4 + 16 p of the wave's range (pass p)
    constexpr int XP = (SPW * kSegs + 15) / 16; // passes of 16 segments
    float xv[XP][8];
    const int nseg = ns * kSegs;
#pragma unroll
    for (int p = 0; p < XP; ++p) {
        const int g = 16 * p + (lane >> 2);
        const int64_t e = s0 * kStep + 32 * (int64_t) g + 8 * (lane & 3);
        if (g < nseg && e < A.K) {
            const float4 u = *reinterpret_cast<const float4 *>(x + e);
            const float4 w = *reinterpret_cast<const float4 *>(x + e + 4);
            xv[p][0] = u.x; xv[p][1] = u.y; xv[p][2] = u.z; xv[p][3] = u.w;
            xv[p][4] = w.x; xv[p][5] = w.y; xv[p][6] = w.z; xv[p][7] = w.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[p][i] = 0.0f;
        }
    }

    F f;
    f.init(A.w[j] + w_off, M, A.nb, g0, rs, lr, part, 0);
    Raw buf[SPW];
#pragma unroll
    for (int i = 0; i < SPW; ++i)
        if (i < ns) buf[i] = f.load(s0 + i);

    XSeg * xs = reinterpret_cast<XSeg *>(lds) + (size_t) wave * SPW * kSegs;
    float4 * xf = reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * SPW * kSegs) + (size_t) wave * SPW * kSegs;
    float * red = reinterpret_cast<float *>(reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * SPW * kSegs) +
                                            (size_t) W * SPW * kSegs);
#pragma unroll
    for (int p = 0; p < XP; ++p) convert_seg(xv[p], 16 * p + (lane >> 2), nseg, lane & 3, xs, xf);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();

    float acc[1] = {0.0f};
    const XView xw{xs, xf, nseg};
#pragma unroll
    for (int i = 0; i < SPW; ++i)
        if (i < ns) f.template compute<1>(buf[i], i * kSegs, xw, acc);

#pragma unroll
    for (int off = R; off < 64; off <<= 1) acc[0] += __shfl_xor(acc[0], off);
    if (part == 0) red[wave * R + r] = acc[0];
    __syncthreads();
    if (tid < R) {
        const int64_t m = m0 + tid;
        if (m < M) {
            float v = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < W; ++w2) v += red[w2 * R + tid];
            A.y[j][i2 * A.y_s2 + i3 * A.y_s3 + m] = v;
        }
    }
}

// One work-group walks tiles blockIdx.x, blockIdx.x + gridDim.x, ... (persistent). Its waves keep
// the same K range for every tile, so each converts its x range once (when the range fits the LDS
// budget; otherwise per chunk of cs steps and tile). The next step's loads (of this tile or the
// first of the next) are in flight while the current step is computed.
template <int DT, int NC, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_mvs(MvArgs A) {
    constexpr int R = 16;
    using F = Fmt<DT, R>;
    using Raw = typename F::Raw;
    extern __shared__ uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane % R, part = lane / R;

    const int64_t sl = blockIdx.y;
    const int64_t i2 = sl % A.ne12, i3 = sl / A.ne12;
    const uint64_t w_off = (uint64_t) (i2 / A.r2) * A.w_s2 + (uint64_t) (i3 / A.r3) * A.w_s3;
    const float * x = A.x + i2 * A.x_s2 + i3 * A.x_s3;

    // the lane's row of a tile (dead lanes of a partial last tile read a real row and drop it)
    struct Row {
        int j;
        int64_t M, m0;
    };
    auto row_of = [&](int64_t tile, F & f) -> Row {
        const int j = tile >= A.tstart[1] ? (tile >= A.tstart[2] ? 2 : 1) : 0;
        const int64_t M = A.M[j];
        const int64_t m0 = (tile - A.tstart[j]) * R;
        const int64_t g0 = m0 & ~(int64_t) 31;
        const int rs = (int) min<int64_t>(32, M - g0);
        const int lr = m0 + r < M ? (int) (m0 - g0) + r : rs - 1;
        f.init(A.w[j] + w_off, M, A.nb, g0, rs, lr, part, 0);
        return Row{j, M, m0};
    };

    // this wave's steps, the same for every tile
    const int64_t s0 = A.nst * wave / W, s1 = A.nst * (wave + 1) / W;
    const int ns = (int) (s1 - s0);
    const int cs = A.cs;
    const bool once = cs >= ns;
    XSeg * xs = reinterpret_cast<XSeg *>(lds) + (size_t) wave * cs * kSegs * NC;
    float4 * xf = reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * cs * kSegs * NC) + (size_t) wave * cs * kSegs * NC;
    float * red = reinterpret_cast<float *>(reinterpret_cast<float4 *>(reinterpret_cast<XSeg *>(lds) + (size_t) W * cs * kSegs * NC) +
                                            (size_t) W * cs * kSegs * NC); // [2][W][NC][R]

    int64_t tile = blockIdx.x;
    F f, fn;
    Row row = row_of(tile, f);
    // two steps in registers: the next step's loads (possibly of the next tile) are issued before
    // the current step's math
    Raw cur;
    if (ns > 0) cur = f.load(s0);
    if (once && ns > 0) convert_x<NC>(A, x, s0 * kStep, ns * kSegs, lane, xs, xf);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();

    for (int it = 0; tile < A.tiles; ++it) {
        const int64_t ntile = tile + gridDim.x;
        const bool has_n = ntile < A.tiles;
        Row nrow{};
        if (has_n) nrow = row_of(ntile, fn);

        float acc[NC];
#pragma unroll
        for (int n = 0; n < NC; ++n) acc[n] = 0.0f;
        for (int k = 0; k < ns; ++k) {
            if (!once && k % cs == 0) {
                // a new x chunk: steps [k, k + cs) of this wave
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                convert_x<NC>(A, x, (s0 + k) * kStep, min(cs, ns - k) * kSegs, lane, xs, xf);
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                __builtin_amdgcn_wave_barrier();
            }
            Raw nxt;
            if (k + 1 < ns) {
                nxt = f.load(s0 + k + 1);
            } else if (has_n) {
                nxt = fn.load(s0);
            }
            const XView xv{xs, xf, min(cs, ns - (k / cs) * cs) * kSegs};
            f.template compute<NC>(cur, (k % cs) * kSegs, xv, acc);
            cur = nxt;
        }

        // parts of a row (lanes r, r + R, ...), then the waves in order
#pragma unroll
        for (int off = R; off < 64; off <<= 1) {
#pragma unroll
            for (int n = 0; n < NC; ++n) acc[n] += __shfl_xor(acc[n], off);
        }
        float * rb = red + (it & 1) * (W * NC * R);
        if (part == 0) {
#pragma unroll
            for (int n = 0; n < NC; ++n) rb[(wave * NC + n) * R + r] = acc[n];
        }
        __syncthreads();
        if (tid < NC * R) {
            const int n = tid / R, rr = tid % R;
            const int64_t m = row.m0 + rr;
            if (m < row.M) {
                float v = 0.0f;
#pragma unroll
                for (int w2 = 0; w2 < W; ++w2) v += rb[(w2 * NC + n) * R + rr];
                A.y[row.j][i2 * A.y_s2 + i3 * A.y_s3 + n * A.ys1[row.j] + m] = v;
            }
        }
        tile = ntile;
        row = nrow;
        f = fn;
    }
}

template <int DT, int R>
void * pick_burst_r(int W, int spw) {
    if (spw <= 2) return W >= 16 ? (void *) k_mvb<DT, R, 16, 2> : W >= 8 ? (void *) k_mvb<DT, R, 8, 2> : (void *) k_mvb<DT, R, 4, 2>;
    return W >= 16 ? (void *) k_mvb<DT, R, 16, 4> : W >= 8 ? (void *) k_mvb<DT, R, 8, 4> : (void *) k_mvb<DT, R, 4, 4>;
}

template <int DT>
void * pick_burst(int W, int spw, int R) {
    if constexpr (DT == Q6_K || DT == Q8_0) {
        if (R == 32 && spw <= 2) return W >= 16 ? (void *) k_mvb<DT, 32, 16, 2> : W >= 8 ? (void *) k_mvb<DT, 32, 8, 2> : (void *) k_mvb<DT, 32, 4, 2>;
        return pick_burst_r<DT, 16>(W, spw);
    } else {
        return R == 32 ? pick_burst_r<DT, 32>(W, spw) : pick_burst_r<DT, 16>(W, spw);
    }
}

// streaming variants: W = 8 for one column, 4 for several
template <int DT>
void * pick(int nc) {
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

} // namespace

hipError_t launch_matvec(const MatArgs * mats, int nmat, int cu_count, hipStream_t stream, const char ** kernel_name,
                          uint64_t * grid_size) {
    constexpr int R = 16;
    if (nmat < 1 || nmat > 3) return hipErrorInvalidValue;
    const MatArgs & a = mats[0];
    for (int j = 0; j < nmat; ++j) {
        if (mats[j].dtype != a.dtype || mats[j].K != a.K || mats[j].N != a.N || (nmat > 1 && mats[j].ne12 * mats[j].ne13 != 1)) {
            return hipErrorInvalidValue;
        }
    }
    const int nc = (int) a.N;
    if (nc < 1 || nc > 8 || a.K <= 0 || a.K % 32 != 0) return hipErrorInvalidValue;
    const int64_t slices = a.ne12 * a.ne13;
    if (slices < 1 || slices > 65535) return hipErrorInvalidValue;
    const int dt = a.dtype;
    if (dt != Q4_0 && dt != Q8_0 && dt != Q4_K && dt != Q6_K) return hipErrorInvalidValue;
    int64_t rows = 0;
    for (int j = 0; j < nmat; ++j) rows += mats[j].M;

    MvArgs L;
    L.tstart[0] = 0;
    for (int j = 0; j < 3; ++j) {
        const bool has = j < nmat;
        L.w[j] = has ? mats[j].w : nullptr;
        L.M[j] = has ? mats[j].M : 0;
        L.y[j] = has ? mats[j].y : nullptr;
        L.ys1[j] = has ? mats[j].y_s1 : 0;
        L.tstart[j + 1] = L.tstart[j] + (has ? (mats[j].M + R - 1) / R : 0);
    }
    for (int j = nmat + 1; j < 4; ++j) L.tstart[j] = INT64_MAX;
    const int64_t tiles = L.tstart[nmat];
    if (tiles < 1 || tiles > 0x7FFFFFFF) return hipErrorInvalidValue;
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
    L.tiles = tiles;

    // burst form (one column, K <= 64 steps): every wave's steps (<= 4) loaded at once, one tile
    // per work-group. 32-row tiles for large products (fewer x conversions per weight, 512-byte
    // runs), 16-row tiles otherwise (more work-groups). 2 steps per wave up to K = 16 steps, then
    // 4 (the 32-row Q6_K / Q8_0 forms hold too many registers at 4 steps: 16 rows there).
    if (nc == 1 && L.xvec && nst <= 64 && tuning("SCRAPGPU_HIP_MV_BURST", 1)) {
        int Rb = rows * slices >= (int64_t) 64 * cu_count ? 32 : 16;
        const int sp = nst <= 32 ? 2 : 4;
        int Wb = 4;
        while (Wb < 16 && (nst + Wb - 1) / Wb > sp) Wb *= 2;
        if (sp == 4 && (dt == Q6_K || dt == Q8_0)) Rb = 16;
        if (const int fr = tuning("SCRAPGPU_HIP_MV_R", 0)) Rb = fr == 32 ? 32 : 16;
        L.tstart[0] = 0;
        for (int j = 0; j < 3; ++j) L.tstart[j + 1] = j < nmat ? L.tstart[j] + (mats[j].M + Rb - 1) / Rb : INT64_MAX;
        const int64_t btiles = L.tstart[nmat];
        L.tiles = btiles;
        L.cs = sp;
        const size_t lds = (size_t) Wb * sp * kSegs * (sizeof(XSeg) + sizeof(float4)) + (size_t) Wb * Rb * sizeof(float);
        void * fn = dt == Q4_0 ? pick_burst<Q4_0>(Wb, sp, Rb) : dt == Q8_0 ? pick_burst<Q8_0>(Wb, sp, Rb)
                  : dt == Q4_K ? pick_burst<Q4_K>(Wb, sp, Rb) : pick_burst<Q6_K>(Wb, sp, Rb);
        if (kernel_name) *kernel_name = name_of(dt, nmat);
        if (grid_size) *grid_size = (uint64_t) btiles * (uint64_t) slices;
        void * args[] = {&L};
        return hipLaunchKernel(fn, dim3((unsigned) btiles, (unsigned) slices), dim3((unsigned) (64 * Wb)), args, lds, stream);
    }

    // streaming form (several columns, or K too long for the burst form)
    const int W = nc == 1 ? 8 : 4;
    // x chunk per wave: all of the wave's steps when they fit the LDS budget, else as many as fit
    const int64_t step_bytes = (int64_t) kSegs * nc * (sizeof(XSeg) + sizeof(float4));
    const int64_t per_wave = std::max<int64_t>(1, (nst + W - 1) / W);
    const int64_t cs = std::min<int64_t>(per_wave, std::max<int64_t>(1, kLdsX / W / step_bytes));
    L.cs = (int) cs;
    const size_t lds = (size_t) W * cs * step_bytes + (size_t) 2 * W * nc * R * sizeof(float);
    if (lds > (size_t) 160 * 1024) return hipErrorInvalidValue;
    void * fn = dt == Q4_0 ? pick<Q4_0>(nc) : dt == Q8_0 ? pick<Q8_0>(nc) : dt == Q4_K ? pick<Q4_K>(nc) : pick<Q6_K>(nc);

    // persistent grid: as many work-groups as stay resident (at most one per tile), trimmed so
    // that every work-group gets the same number of tiles
    const int per_cu = std::max(1, tuning("SCRAPGPU_HIP_MV_WGS", occupancy(fn, 64 * W, lds)));
    const int64_t cap = std::max<int64_t>(1, (int64_t) per_cu * cu_count / slices);
    const int64_t rounds = (tiles + cap - 1) / cap;
    const int64_t grid_x = (tiles + rounds - 1) / rounds;

    if (kernel_name) *kernel_name = name_of(dt, nmat);
    if (grid_size) *grid_size = (uint64_t) grid_x * (uint64_t) slices;
    void * args[] = {&L};
    return hipLaunchKernel(fn, dim3((unsigned) grid_x, (unsigned) slices), dim3((unsigned) (64 * W)), args, lds, stream);
}

} // namespace sgk
