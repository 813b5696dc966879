// Decode matvec over R32 weights for 1 <= N <= 8 columns (gfx950, wave64).
//
// Work decomposition. A work-group owns R consecutive rows (a whole R32 group or an aligned part
// of one) of one slice and the whole K range, so no work-group ever waits for
// another: on MI355X the 8 XCDs have separate L2s and any cross-work-group handshake inside a
// kernel costs an L2 write-back/invalidate. R (32, 16, 8 or 4) is picked per shape so that the grid
// holds at least two work-groups per CU. Its W waves (8, up to 16 for small grids) split K: wave w
// takes steps w, w+W, ...; each wave keeps 4 steps of weight loads in flight in a register ring,
// and issues the first ones before the x chunk is staged so that the two overlap.
//
// Inside a wave, lane l serves row r = l % R of the tile through slot s = l / R (S = 64 / R slots).
// A step covers `bps` blocks whose "tasks" (16-byte R32 units, or for Q6_K the three units that
// hold one 64-element run) are dealt to the slots, so one wave-wide 128-bit load reads S runs of
// 16*R contiguous bytes (>= 64 bytes): coalesced.
//
// Arithmetic. A lane converts bytes with one mask per 4 weights and one byte->float conversion per
// weight, then one FMA per weight and column against x held in LDS (lanes of a slot read the same
// LDS address: a broadcast). Block scales are factored out of the inner sums and every constant
// offset of a format is applied once per 16 weights through precomputed sums of 16 consecutive x:
//   Q4_0: d * (sum q x - 8 sum x)            Q8_0: d * (sum u x - 128 sum x)   (u = q xor 0x80)
//   Q4_K: d*sc * sum q x - dmin*m * sum x    Q6_K: d*sc * (sum q x - 32 sum x)
// The high nibble is used in place (value * 16) and the 1/16 folded into its scale. The slots and
// then the waves of a row are added in a fixed order (shuffles, then LDS): deterministic.
//
// x is staged per K chunk (all of K when it fits the LDS budget, else chunks of whole steps).
#include "kernels.h"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <vector>

namespace sgk {
namespace {

constexpr int kMaxWaves = 8;
constexpr int kDepth = 4;      // most steps in flight per wave
constexpr int kLdsBudget = 56 * 1024; // bytes of x (+ sums) per work-group

struct MvLaunch {
    MatArgs a;          // K, nb, x, slices and strides (w / M / y per matrix below)
    int64_t tiles;      // row tiles per slice, over all matrices
    int64_t kc;         // K elements staged per chunk (a multiple of the step)
    int wt;             // waves that split the K steps of one tile
    int nmat;           // 1, or 2..3 weights sharing x (MUL_MAT_MULTI)
    const uint8_t * wm[3];
    int64_t Mm[3];
    float * ym[3];
    int64_t ys1[3];
    int64_t tstart[4];  // matrix j owns tiles [tstart[j], tstart[j + 1])
};

__device__ __forceinline__ float half_bits(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short) (h & 0xFFFFu)));
}

__device__ __forceinline__ uint4 mask4(uint4 q, uint32_t m) {
    return make_uint4(q.x & m, q.y & m, q.z & m, q.w & m);
}

__device__ __forceinline__ uint4 load16(const uint8_t * p) {
    return *reinterpret_cast<const uint4 *>(p);
}

__device__ __forceinline__ uint32_t byte_of(uint4 v, int i) {
    const uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return (w >> (8 * (i & 3))) & 0xFFu;
}

// steps in flight per wave: the largest power of two (<= kDepth) whose raw weight registers fit in
// ~48 VGPRs; the host picks the waves per tile so that every wave's step count is a multiple of it
constexpr int ring_depth(size_t raw_bytes) {
    return (int) (raw_bytes / 4) * 4 <= 48 ? 4 : (int) (raw_bytes / 4) * 2 <= 48 ? 2 : 1;
}

// ---- per format: tasks per block, elements per block, raw registers of one task ----------------

// The x chunk in LDS: for column n and 16-element segment g, xq[(n * nseg + g)] holds two int8
// planes (a, b) with x ~= s * a + (s / 256) * b, and xf[(n * nseg + g)] = {s / 256, sum of the 16 x}.
struct XSeg {
    uint4 a, b;
};

// 256 * sum(q_i * a_i) + sum(q_i * b_i) over 16 int8 pairs: x dot q in units of s / 256
__device__ __forceinline__ int dot16i(uint4 q, const XSeg & x) {
    int t = __builtin_amdgcn_sdot4((int) q.x, (int) x.a.x, 0, false);
    t = __builtin_amdgcn_sdot4((int) q.y, (int) x.a.y, t, false);
    t = __builtin_amdgcn_sdot4((int) q.z, (int) x.a.z, t, false);
    t = __builtin_amdgcn_sdot4((int) q.w, (int) x.a.w, t, false);
    t <<= 8;
    t = __builtin_amdgcn_sdot4((int) q.x, (int) x.b.x, t, false);
    t = __builtin_amdgcn_sdot4((int) q.y, (int) x.b.y, t, false);
    t = __builtin_amdgcn_sdot4((int) q.z, (int) x.b.z, t, false);
    t = __builtin_amdgcn_sdot4((int) q.w, (int) x.b.w, t, false);
    return t;
}

__device__ __forceinline__ uint4 shr4(uint4 q, int s) {
    return make_uint4(q.x >> s, q.y >> s, q.z >> s, q.w >> s);
}

// ---- per format: the lane's view of one row tile ------------------------------------------------
// A Stepper is built once per tile: 64-bit base pointers of the lane's row in every R32 area, then
// 32-bit offsets per step. load(step) fetches all the lane's 16-byte units of one step (and the
// block's scales once); compute() accumulates them against x.

template <int DT, int R> struct Stepper;

// blocks per step, tasks per lane and step, K elements per step of a format with T tasks per block
template <int T, int R, int BE>
struct Geo {
    static constexpr int S = 64 / R;
    static constexpr int BPS = S > T ? S / T : 1;
    static constexpr int TPL = T * BPS / S;
    static constexpr int EPS = BPS * BE;
};

template <int R>
struct Stepper<Q4_0, R> : Geo<1, R, 32> {
    using G = Geo<1, R, 32>;
    struct Raw { uint4 q; uint32_t d; };
    const uint8_t * qb;
    const uint8_t * db;
    uint32_t qblk, dblk;
    int64_t nb;
    int slot;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb_, int64_t g0, int rs, int lr, int slot_) {
        nb = nb_;
        slot = slot_;
        qb = w + (uint64_t) g0 * nb * 16 + (uint64_t) lr * 16;
        db = w + (uint64_t) M * nb * 16 + (uint64_t) g0 * nb * 2 + (uint64_t) lr * 2;
        qblk = (uint32_t) rs * 16;
        dblk = (uint32_t) rs * 2;
    }
    __device__ int64_t block(int64_t step) const { return step * G::BPS + slot; }
    __device__ Raw load(int64_t step) const {
        Raw r{};
        const int64_t b = block(step);
        if (b < nb) {
            r.q = load16(qb + (uint32_t) b * qblk);
            r.d = *reinterpret_cast<const uint16_t *>(db + (uint32_t) b * dblk);
        }
        return r;
    }
    template <int NC>
    __device__ void compute(const Raw & r, int64_t step, int64_t kc0, const XSeg * xq, const float2 * xf, int nseg, float * acc) const {
        const int64_t b = block(step);
        if (b >= nb) return;
        const int sg = (int) ((b * 32 - kc0) >> 4);
        const float d = half_bits(r.d);
        const uint4 lo = mask4(r.q, 0x0F0F0F0Fu), hi = mask4(shr4(r.q, 4), 0x0F0F0F0Fu);
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            const int g = n * nseg + sg;
            const float2 f0 = xf[g], f1 = xf[g + 1];
            float a = acc[n];
            a = fmaf(d * f0.x, (float) dot16i(lo, xq[g]), a);
            a = fmaf(d * f1.x, (float) dot16i(hi, xq[g + 1]), a);
            a = fmaf(-8.0f * d, f0.y + f1.y, a);
            acc[n] = a;
        }
    }
};

template <int R>
struct Stepper<Q8_0, R> : Geo<2, R, 32> {
    using G = Geo<2, R, 32>;
    struct Raw { uint4 q; uint32_t d; };
    const uint8_t * qb;
    const uint8_t * db;
    uint32_t qblk, qunit, dblk;
    int64_t nb;
    int slot;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb_, int64_t g0, int rs, int lr, int slot_) {
        nb = nb_;
        slot = slot_;
        qb = w + (uint64_t) g0 * nb * 32 + (uint64_t) lr * 16;
        db = w + (uint64_t) M * nb * 32 + (uint64_t) g0 * nb * 2 + (uint64_t) lr * 2;
        qblk = (uint32_t) rs * 32;
        qunit = (uint32_t) rs * 16;
        dblk = (uint32_t) rs * 2;
    }
    // TPL == 1: the lane's task is slot -> block step * BPS + slot / 2, unit slot % 2
    __device__ int64_t block(int64_t step) const { return step * G::BPS + slot / 2; }
    __device__ Raw load(int64_t step) const {
        Raw r{};
        const int64_t b = block(step);
        if (b < nb) {
            r.q = load16(qb + (uint32_t) b * qblk + (uint32_t) (slot & 1) * qunit);
            r.d = *reinterpret_cast<const uint16_t *>(db + (uint32_t) b * dblk);
        }
        return r;
    }
    template <int NC>
    __device__ void compute(const Raw & r, int64_t step, int64_t kc0, const XSeg * xq, const float2 * xf, int nseg, float * acc) const {
        const int64_t b = block(step);
        if (b >= nb) return;
        const int sg = (int) ((b * 32 - kc0) >> 4) + (slot & 1);
        const float d = half_bits(r.d);
        const uint4 q = make_uint4(r.q.x ^ 0x80808080u, r.q.y ^ 0x80808080u, r.q.z ^ 0x80808080u, r.q.w ^ 0x80808080u);
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            const int g = n * nseg + sg;
            acc[n] = fmaf(d * xf[g].x, (float) dot16i(q, xq[g]), acc[n]);
        }
    }
};

// 6-bit scale and min of sub-block j (0..7) from the 12 packed bytes s[0..11] = {hd.y, hd.z, hd.w}
__device__ __forceinline__ void k4_scale_min(uint4 hd, int j, float & sc, float & mn) {
    const uint32_t lo4 = hd.y, hi4 = hd.z, top4 = hd.w; // s[0..3], s[4..7], s[8..11]
    const int sh = 8 * (j & 3);
    if (j < 4) {
        sc = (float) ((lo4 >> sh) & 63u);
        mn = (float) ((hi4 >> sh) & 63u);
    } else {
        const uint32_t t = (top4 >> sh) & 0xFFu;
        sc = (float) ((t & 0x0Fu) | (((lo4 >> sh) >> 6 & 3u) << 4));
        mn = (float) ((t >> 4) | (((hi4 >> sh) >> 6 & 3u) << 4));
    }
}

template <int R>
struct Stepper<Q4_K, R> : Geo<8, R, 256> {
    using G = Geo<8, R, 256>;
    struct Raw { uint4 q[G::TPL]; uint4 hd; };
    const uint8_t * qb;
    const uint8_t * hb;
    uint32_t qblk, qunit, hblk;
    int slot;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb, int64_t g0, int rs, int lr, int slot_) {
        slot = slot_;
        qb = w + (uint64_t) g0 * nb * 128 + (uint64_t) lr * 16;
        hb = w + (uint64_t) M * nb * 128 + (uint64_t) g0 * nb * 16 + (uint64_t) lr * 16;
        qblk = (uint32_t) rs * 128;
        qunit = (uint32_t) rs * 16;
        hblk = (uint32_t) rs * 16;
    }
    __device__ Raw load(int64_t step) const {
        Raw r;
        const uint8_t * p = qb + (uint32_t) step * qblk + (uint32_t) slot * qunit;
#pragma unroll
        for (int t = 0; t < G::TPL; ++t) r.q[t] = load16(p + (uint32_t) (G::S * t) * qunit);
        r.hd = load16(hb + (uint32_t) step * hblk);
        return r;
    }
    template <int NC>
    __device__ void compute(const Raw & r, int64_t step, int64_t kc0, const XSeg * xq, const float2 * xf, int nseg, float * acc) const {
        const float d = half_bits(r.hd.x), dmin = half_bits(r.hd.x >> 16);
        const int sg0 = (int) ((step * 256 - kc0) >> 4);
#pragma unroll
        for (int t = 0; t < G::TPL; ++t) {
            const int j = slot + G::S * t; // unit: bytes 16j..16j+15 of the 128 quant bytes
            const int c = j >> 1, h = j & 1;
            float sc0, m0, sc1, m1;
            k4_scale_min(r.hd, 2 * c, sc0, m0);
            k4_scale_min(r.hd, 2 * c + 1, sc1, m1);
            const float dl = d * sc0, dh = d * sc1, ml = dmin * m0, mh = dmin * m1;
            const uint4 lo = mask4(r.q[t], 0x0F0F0F0Fu), hi = mask4(shr4(r.q[t], 4), 0x0F0F0F0Fu);
            const int sg = sg0 + 4 * c + h; // lo elements 64c + 16h + i, hi 32 further
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                const int g = n * nseg + sg;
                const float2 fl = xf[g], fh = xf[g + 2];
                float a = acc[n];
                a = fmaf(dl * fl.x, (float) dot16i(lo, xq[g]), a);
                a = fmaf(dh * fh.x, (float) dot16i(hi, xq[g + 2]), a);
                a = fmaf(-ml, fl.y, a);
                a = fmaf(-mh, fh.y, a);
                acc[n] = a;
            }
        }
    }
};

template <int R>
struct Stepper<Q6_K, R> : Geo<4, R, 256> {
    using G = Geo<4, R, 256>;
    struct Raw { uint4 qa[G::TPL], qc[G::TPL], qh[G::TPL]; uint4 sc; uint32_t d; };
    const uint8_t * qb;
    const uint8_t * sb;
    const uint8_t * db;
    uint32_t qblk, qunit, sblk, dblk;
    int64_t nb;
    int slot;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb_, int64_t g0, int rs, int lr, int slot_) {
        nb = nb_;
        slot = slot_;
        qb = w + (uint64_t) g0 * nb * 192 + (uint64_t) lr * 16;
        sb = w + (uint64_t) M * nb * 192 + (uint64_t) g0 * nb * 16 + (uint64_t) lr * 16;
        db = w + (uint64_t) M * nb * 208 + (uint64_t) g0 * nb * 2 + (uint64_t) lr * 2;
        qblk = (uint32_t) rs * 192;
        qunit = (uint32_t) rs * 16;
        sblk = (uint32_t) rs * 16;
        dblk = (uint32_t) rs * 2;
    }
    // task k = 0..3: h = k >> 1 (half of the block), hf = k & 1 (16-element half of each 32-run)
    __device__ int task(int t) const { return (slot + G::S * t) % 4; }
    __device__ int64_t block(int64_t step) const { return step * G::BPS + (G::BPS > 1 ? slot / 4 : 0); }
    __device__ Raw load(int64_t step) const {
        Raw r{};
        const int64_t b = block(step);
        if (G::BPS > 1 && b >= nb) return r;
        const uint8_t * p = qb + (uint32_t) b * qblk;
#pragma unroll
        for (int t = 0; t < G::TPL; ++t) {
            const int k = task(t), h = k >> 1, hf = k & 1;
            r.qa[t] = load16(p + (uint32_t) (4 * h + hf) * qunit);     // ql[64h + 16hf + i]
            r.qc[t] = load16(p + (uint32_t) (4 * h + 2 + hf) * qunit); // ql[64h + 32 + 16hf + i]
            r.qh[t] = load16(p + (uint32_t) (8 + 2 * h + hf) * qunit); // qh[32h + 16hf + i]
        }
        r.sc = load16(sb + (uint32_t) b * sblk);
        r.d = *reinterpret_cast<const uint16_t *>(db + (uint32_t) b * dblk);
        return r;
    }
    template <int NC>
    __device__ void compute(const Raw & r, int64_t step, int64_t kc0, const XSeg * xq, const float2 * xf, int nseg, float * acc) const {
        const int64_t b = block(step);
        if (G::BPS > 1 && b >= nb) return;
        const float d = half_bits(r.d);
        const int sg0 = (int) ((b * 256 - kc0) >> 4);
#pragma unroll
        for (int t = 0; t < G::TPL; ++t) {
            const int k = task(t), h = k >> 1, hf = k & 1;
            const uint4 qa = r.qa[t], qc = r.qc[t], qh = r.qh[t];
            uint4 v[4];
            v[0] = make_uint4((qa.x & 0x0F0F0F0Fu) | ((qh.x << 4) & 0x30303030u), (qa.y & 0x0F0F0F0Fu) | ((qh.y << 4) & 0x30303030u),
                              (qa.z & 0x0F0F0F0Fu) | ((qh.z << 4) & 0x30303030u), (qa.w & 0x0F0F0F0Fu) | ((qh.w << 4) & 0x30303030u));
            v[1] = make_uint4((qc.x & 0x0F0F0F0Fu) | ((qh.x << 2) & 0x30303030u), (qc.y & 0x0F0F0F0Fu) | ((qh.y << 2) & 0x30303030u),
                              (qc.z & 0x0F0F0F0Fu) | ((qh.z << 2) & 0x30303030u), (qc.w & 0x0F0F0F0Fu) | ((qh.w << 2) & 0x30303030u));
            v[2] = make_uint4(((qa.x >> 4) & 0x0F0F0F0Fu) | (qh.x & 0x30303030u), ((qa.y >> 4) & 0x0F0F0F0Fu) | (qh.y & 0x30303030u),
                              ((qa.z >> 4) & 0x0F0F0F0Fu) | (qh.z & 0x30303030u), ((qa.w >> 4) & 0x0F0F0F0Fu) | (qh.w & 0x30303030u));
            v[3] = make_uint4(((qc.x >> 4) & 0x0F0F0F0Fu) | ((qh.x >> 2) & 0x30303030u), ((qc.y >> 4) & 0x0F0F0F0Fu) | ((qh.y >> 2) & 0x30303030u),
                              ((qc.z >> 4) & 0x0F0F0F0Fu) | ((qh.z >> 2) & 0x30303030u), ((qc.w >> 4) & 0x0F0F0F0Fu) | ((qh.w >> 2) & 0x30303030u));
            // scale byte 8h + 2rr + hf (stored xor 0x80): the 4 bytes for rr = 0..3 are
            // s[8h + hf], s[8h + hf + 2], ... -> word h*2 + (hf? odd bytes) of sc
            const uint32_t sw0 = h ? r.sc.z : r.sc.x, sw1 = h ? r.sc.w : r.sc.y; // bytes 8h..8h+3, 8h+4..8h+7
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const uint32_t sw = rr < 2 ? sw0 : sw1;
                const int bi = 2 * (rr & 1) + hf;
                const float ds = d * (float) (int8_t) (((sw >> (8 * bi)) & 0xFFu) ^ 0x80u);
                const int sg = sg0 + 8 * h + 2 * rr + hf; // elements 128h + 32rr + 16hf + i
#pragma unroll
                for (int n = 0; n < NC; ++n) {
                    const int g = n * nseg + sg;
                    const float2 f = xf[g];
                    float a = acc[n];
                    a = fmaf(ds * f.x, (float) dot16i(v[rr], xq[g]), a);
                    a = fmaf(-32.0f * ds, f.y, a);
                    acc[n] = a;
                }
            }
        }
    }
};

template <int DT, int NC, int R>
__global__ __launch_bounds__(64 * kMaxWaves) void k_matvec(MvLaunch L) {
    using ST = Stepper<DT, R>;
    using Raw = typename ST::Raw;
    constexpr int S = ST::S;
    constexpr int EPS = ST::EPS;
    constexpr int D = ring_depth(sizeof(Raw)); // steps in flight per wave
    extern __shared__ float lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int W = blockDim.x >> 6;
    const int WT = L.wt;                  // waves per tile
    const int GW = W / WT;                // tiles in flight per work-group
    const int grp = wave / WT, wt = wave % WT;
    const int r = lane % R, slot = lane / R;
    const int64_t sl = blockIdx.y;
    const int64_t i2 = sl % L.a.ne12, i3 = sl / L.a.ne12;
    const int64_t K = L.a.K;
    const uint64_t w_off = (uint64_t) (i2 / L.a.r2) * L.a.w_s2 + (uint64_t) (i3 / L.a.r3) * L.a.w_s3;
    const int64_t y_off = i2 * L.a.y_s2 + i3 * L.a.y_s3;
    const float * x = L.a.x + i2 * L.a.x_s2 + i3 * L.a.x_s3;
    // matrix of a tile (tiles of matrix j are [tstart[j], tstart[j + 1]))
    auto mat_of = [&](int64_t tile) { return tile >= L.tstart[1] ? (tile >= L.tstart[2] ? 2 : 1) : 0; };
    // tiles of this work-group: iteration it, group g -> tile (it * gridDim.x + blockIdx.x) * GW + g
    const int64_t per_iter = (int64_t) gridDim.x * GW;
    const int64_t iters = (L.tiles + per_iter - 1) / per_iter;
    auto tile_of = [&](int64_t it) { return (it * gridDim.x + blockIdx.x) * GW + grp; };
    // the lane's addressing for the tile of iteration it (live: its row exists)
    auto stepper_of = [&](int64_t it, ST & st) -> bool {
        const int64_t tile = tile_of(it);
        if (tile >= L.tiles) return false;
        const int j = mat_of(tile);
        const int64_t M = L.Mm[j], m0 = (tile - L.tstart[j]) * R;
        if (m0 + r >= M) return false;
        const int64_t g0 = m0 & ~(int64_t) 31;
        st.init(L.wm[j] + w_off, M, L.a.nb, g0, (int) min<int64_t>(32, M - g0), (int) (m0 - g0) + r, slot);
        return true;
    };

    Raw ring[D];
    ST cur, nxt;

    for (int64_t kc0 = 0; kc0 < K; kc0 += L.kc) {
        const int xlen = (int) min<int64_t>(L.kc, K - kc0);
        const int64_t st0 = kc0 / EPS;
        const int nst = (int) ((kc0 + xlen + EPS - 1) / EPS - st0); // steps of this chunk
        const int nw = wt < nst ? (nst - wt + WT - 1) / WT : 0;      // this wave's steps per tile
        const int nwp = (nw + D - 1) / D * D;                        // padded to whole ring turns
        bool live = stepper_of(0, cur);
        bool live_n = stepper_of(1, nxt);
        // weight loads first: they do not depend on x and overlap the staging below
        if (live) {
#pragma unroll
            for (int j = 0; j < D; ++j)
                if (j < nw) ring[j] = cur.load(st0 + wt + (int64_t) WT * j);
        }

        const int nseg = xlen / 16;
        XSeg * xq = reinterpret_cast<XSeg *>(lds);
        float2 * xf = reinterpret_cast<float2 *>(xq + NC * nseg);
        float * red = reinterpret_cast<float *>(xf + NC * nseg); // [2][W][NC][R]
        __syncthreads(); // the previous chunk is consumed
        // one thread per (column, segment): two int8 planes, the plane scale and the plain sum
        for (int i = tid; i < NC * nseg; i += blockDim.x) {
            const int n = i / nseg, sg = i - n * nseg;
            const float * xp = x + n * L.a.x_s1 + kc0 + 16 * sg;
            float v[16];
            float amax = 0.0f, sum = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                v[e] = xp[e];
                amax = fmaxf(amax, fabsf(v[e]));
                sum += v[e];
            }
            const float s1 = amax * (1.0f / 127.0f);
            const float inv1 = amax > 0.0f ? 127.0f / amax : 0.0f;
            uint32_t pa[4] = {0, 0, 0, 0}, pb[4] = {0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float qa = fminf(127.0f, fmaxf(-127.0f, rintf(v[e] * inv1)));
                const float res = fmaf(-qa, s1, v[e]);
                const float qb = fminf(127.0f, fmaxf(-127.0f, rintf(res * (256.0f * inv1))));
                pa[e >> 2] |= ((uint32_t) (int) qa & 0xFFu) << (8 * (e & 3));
                pb[e >> 2] |= ((uint32_t) (int) qb & 0xFFu) << (8 * (e & 3));
            }
            XSeg xs_;
            xs_.a = make_uint4(pa[0], pa[1], pa[2], pa[3]);
            xs_.b = make_uint4(pb[0], pb[1], pb[2], pb[3]);
            xq[i] = xs_;
            xf[i] = make_float2(s1 * (1.0f / 256.0f), sum);
        }
        __syncthreads();

        for (int64_t it = 0; it < iters; ++it) {
            float acc[NC];
#pragma unroll
            for (int n = 0; n < NC; ++n) acc[n] = 0.0f;
            for (int i = 0; i < nwp; i += D) {
#pragma unroll
                for (int j = 0; j < D; ++j) {
                    const int ii = i + j;
                    if (live && ii < nw) cur.template compute<NC>(ring[j], st0 + wt + (int64_t) WT * ii, kc0, xq, xf, nseg, acc);
                    // refill this ring slot with the item D ahead (possibly of the next tile)
                    const int ni = ii + D;
                    if (ni < nwp) {
                        if (live && ni < nw) ring[j] = cur.load(st0 + wt + (int64_t) WT * ni);
                    } else if (live_n && ni - nwp < nw) {
                        ring[j] = nxt.load(st0 + wt + (int64_t) WT * (ni - nwp));
                    }
                }
            }
            // slots of a row: lanes r, r + R, ... (fixed butterfly order)
#pragma unroll
            for (int off = R; off < 64; off <<= 1) {
#pragma unroll
                for (int n = 0; n < NC; ++n) acc[n] += __shfl_xor(acc[n], off);
            }
            float * rb = red + (it & 1) * (W * NC * R);
            if (slot == 0) {
#pragma unroll
                for (int n = 0; n < NC; ++n) rb[(wave * NC + n) * R + r] = acc[n];
            }
            __syncthreads();
            if (tid < GW * NC * R) {
                const int g = tid / (NC * R), n = (tid / R) % NC, rr = tid % R;
                const int64_t t2 = (it * gridDim.x + blockIdx.x) * GW + g;
                const int jm = mat_of(t2);
                const int64_t m = (t2 - L.tstart[jm]) * R + rr;
                if (t2 < L.tiles && m < L.Mm[jm]) {
                    float v = 0.0f;
                    for (int w2 = 0; w2 < WT; ++w2) v += rb[((g * WT + w2) * NC + n) * R + rr];
                    float * yp = L.ym[jm] + y_off + n * L.ys1[jm] + m;
                    *yp = kc0 == 0 ? v : *yp + v;
                }
            }
            cur = nxt;
            live = live_n;
            live_n = stepper_of(it + 2, nxt);
        }
    }
}

template <int DT, int R>
void * pick_nc(int nc) {
    switch (nc) {
        case 1: return (void *) k_matvec<DT, 1, R>;
        case 2: return (void *) k_matvec<DT, 2, R>;
        case 3: return (void *) k_matvec<DT, 3, R>;
        case 4: return (void *) k_matvec<DT, 4, R>;
        case 5: return (void *) k_matvec<DT, 5, R>;
        case 6: return (void *) k_matvec<DT, 6, R>;
        case 7: return (void *) k_matvec<DT, 7, R>;
        default: return (void *) k_matvec<DT, 8, R>;
    }
}

template <int DT>
void * pick(int nc, int R) {
    return R == 32 ? pick_nc<DT, 32>(nc) : R == 16 ? pick_nc<DT, 16>(nc) : pick_nc<DT, 8>(nc);
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

// tuning overrides from the environment (read once; 0 / unset = automatic)
int tuning(const char * name, int dflt) {
    const char * v = std::getenv(name);
    return v != nullptr && *v ? std::atoi(v) : dflt;
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

int tasks_of(int dt) {
    return dt == Q4_0 ? 1 : dt == Q8_0 ? 2 : dt == Q4_K ? 8 : 4;
}

template <int R>
size_t raw_bytes_r(int dt) {
    return dt == Q4_0 ? sizeof(typename Stepper<Q4_0, R>::Raw) : dt == Q8_0 ? sizeof(typename Stepper<Q8_0, R>::Raw)
         : dt == Q4_K ? sizeof(typename Stepper<Q4_K, R>::Raw) : sizeof(typename Stepper<Q6_K, R>::Raw);
}

size_t raw_bytes_of(int dt, int R) {
    return R == 32 ? raw_bytes_r<32>(dt) : R == 16 ? raw_bytes_r<16>(dt) : raw_bytes_r<8>(dt);
}

} // namespace

hipError_t launch_matvec(const MatArgs * mats, int nmat, int cu_count, hipStream_t stream, const char ** kernel_name,
                         uint64_t * grid_size) {
    if (nmat < 1 || nmat > 3) return hipErrorInvalidValue;
    const MatArgs & a = mats[0];
    int64_t m_total = 0;
    for (int j = 0; j < nmat; ++j) {
        if (mats[j].dtype != a.dtype || mats[j].K != a.K || mats[j].N != a.N || (nmat > 1 && mats[j].ne12 * mats[j].ne13 != 1)) {
            return hipErrorInvalidValue;
        }
        m_total += mats[j].M;
    }
    const int nc = (int) a.N;
    if (nc < 1 || nc > 8) return hipErrorInvalidValue;
    const int64_t slices = a.ne12 * a.ne13;
    if (slices > 65535) return hipErrorInvalidValue;
    const int T = tasks_of(a.dtype);
    const int be = a.dtype == Q4_K || a.dtype == Q6_K ? 256 : 32;
    // x chunk: as much of K as fits the LDS budget, in whole steps (of the smallest row tile)
    const int eps_max = (64 / 8 > T ? 64 / 8 / T : 1) * be;
    const int64_t max_kc = std::max<int64_t>(eps_max, (int64_t) (kLdsBudget / (3 * nc)) / eps_max * eps_max); // 2 B + 8/16 B per element
    MvLaunch L;
    L.a = a;
    L.kc = std::min<int64_t>(a.K, max_kc);
    // persistent grid: as many 8-wave work-groups as stay resident (occupancy of the chosen kernel
    // with its LDS; SCRAPGPU_HIP_MV_WGS overrides the per-CU count), shared among the slices
    const int waves = kMaxWaves;
    auto pick_fn = [&](int R) -> void * {
        switch (a.dtype) {
            case Q4_0: return pick<Q4_0>(nc, R);
            case Q8_0: return pick<Q8_0>(nc, R);
            case Q4_K: return pick<Q4_K>(nc, R);
            case Q6_K: return pick<Q6_K>(nc, R);
            default: return nullptr;
        }
    };
    auto lds_of = [&](int R) { return (size_t) nc * (L.kc / 16) * (32 + 8) + (size_t) 2 * waves * nc * R * sizeof(float); };
    auto resident = [&](int R) -> int64_t {
        int per_cu = tuning("SCRAPGPU_HIP_MV_WGS", 0);
        if (per_cu <= 0) per_cu = occupancy(pick_fn(R), 64 * waves, lds_of(R));
        return std::max<int64_t>(1, (int64_t) std::max(1, per_cu) * cu_count / slices);
    };
    // row tile: the largest (32, 16, 8) that still gives every wave group >= 2 tiles; the waves of
    // a group split the K steps while each keeps >= 2 ring turns
    int R = 8, WT = 1;
    int64_t wgs = 1;
    for (int cand : {32, 16, 8}) {
        const int S = 64 / cand;
        const int eps = (S > T ? S / T : 1) * be;
        const int D = ring_depth(raw_bytes_of(a.dtype, cand));
        const int64_t nst = (L.kc + eps - 1) / eps;
        int wt = 1;
        while (wt < waves && nst % (2 * wt) == 0 && (nst / (2 * wt)) % D == 0 && nst / (2 * wt) >= 2 * D) wt *= 2;
        int64_t tiles = 0;
        for (int j = 0; j < nmat; ++j) tiles += (mats[j].M + cand - 1) / cand;
        R = cand;
        WT = wt;
        wgs = resident(cand);
        if (tiles >= 2 * wgs * (waves / wt)) break;
    }
    if (const int fr = tuning("SCRAPGPU_HIP_MV_R", 0)) R = fr;
    if (const int fw = tuning("SCRAPGPU_HIP_MV_WT", 0)) WT = fw;
    L.wt = WT;
    L.nmat = nmat;
    L.tstart[0] = 0;
    for (int j = 0; j < 3; ++j) {
        const bool has = j < nmat;
        L.wm[j] = has ? mats[j].w : nullptr;
        L.Mm[j] = has ? mats[j].M : 0;
        L.ym[j] = has ? mats[j].y : nullptr;
        L.ys1[j] = has ? mats[j].y_s1 : 0;
        L.tstart[j + 1] = L.tstart[j] + (has ? (mats[j].M + R - 1) / R : 0);
    }
    for (int j = nmat + 1; j < 4; ++j) L.tstart[j] = INT64_MAX; // tiles past the last matrix never map there
    L.tiles = L.tstart[nmat];
    (void) m_total;
    wgs = resident(R);
    const int64_t grid_x = std::max<int64_t>(1, std::min<int64_t>(wgs, (L.tiles + (waves / WT) - 1) / (waves / WT)));
    const size_t lds = lds_of(R);
    void * fn = pick_fn(R);
    if (fn == nullptr) return hipErrorInvalidValue;
    if (kernel_name) *kernel_name = name_of(a.dtype, nmat);
    if (grid_size) *grid_size = (uint64_t) grid_x * (uint64_t) slices;
    void * args[] = {&L};
    return hipLaunchKernel(fn, dim3((unsigned) grid_x, (unsigned) slices), dim3((unsigned) (64 * waves)), args, lds, stream);
}

} // namespace sgk
