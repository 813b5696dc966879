// Prefill matmul over R32 weights on the bf16 MFMA units of gfx950 (fp32 accumulate), N > 8.
//
// Replaces, for the hip backend, the reference's tiled mat-mat kernels k_mm_* / k_mmx_*
// (src/backends/opencl11/kernels/mul_mm.cl:270-355, mul_mm_x.cl:437-539). Same product, new design:
//
//   pre-pass  x (fp32, any column stride) -> xb (bf16, [slice][N][K] contiguous) in stream scratch,
//             once per op, so the GEMM reads half the activation bytes and converts nothing twice.
//   GEMM      a work-group (4 waves) owns 128 weight rows x 128 tokens and walks K in stages of
//             128. Wave w owns rows 32w .. 32w + 31 (two 16-row groups) and all 128 tokens.
//               * B operand (weights): lane (r, g) of a 16-row group loads, per stage, the R32 units
//                 of row r that hold its 32 codes (one 16-byte unit for Q4_K / Q4_0 / Q8_0-half,
//                 three for Q6_K), dequantizes them in registers (d*sc*q - dmin*m in fp32, packed
//                 to bf16) and feeds 8 of them to each of the stage's 4 MFMA k-steps. No weight
//                 tile goes through LDS: every weight is dequantized exactly once per work-group.
//               * A operand (activations): the 128 x 128 bf16 x tile of the stage, staged in LDS
//                 (double-buffered, XOR-swizzled 16-byte chunks) and read as 8 token fragments per
//                 k-step. The k order inside a step is whatever the weight lanes hold; the A reads
//                 follow it (chunk(g, t) below), which the MFMA allows because its A and B operands
//                 share one k mapping per lane group.
//               * v_mfma_f32_16x16x32_bf16, 2 row groups x 8 token fragments per k-step: each B
//                 fragment serves 8 MFMAs, each A fragment 2.
//             The next stage's weights and x tile are loaded into registers while the current
//             stage computes; one barrier per stage.
//   split-K   when the tiles alone cannot fill the GPU, K is split over work-groups that write
//             partial sums to scratch; a reduction kernel adds them in split order (deterministic).
#include "kernels.h"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdlib>

namespace sgk {
namespace {

constexpr int BM = 128, BK = 128;
constexpr int kThreads = 256;
constexpr int kChunks = BK / 8; // 16-byte chunks per LDS row of the x tile

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// two floats -> two bf16 (round to nearest even) in one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    const bf16x2 v = __builtin_convertvector((f32x2{a, b}), bf16x2);
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float half_bits(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short) (h & 0xFFFFu)));
}

__device__ __forceinline__ uint4 load16(const uint8_t * p) {
    return *reinterpret_cast<const uint4 *>(p);
}

// byte i of w as a float (v_cvt_f32_ubyte<i>: one instruction; the compiler would otherwise
// extract the byte first)
template <int I>
__device__ __forceinline__ float ubyte(uint32_t w) {
    float f;
    if constexpr (I == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(w));
    else if constexpr (I == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(w));
    else if constexpr (I == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(w));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(w));
    return f;
}

// 8 bf16 = scale * byte_i - offset for the bytes of words w0, w1 (byte values 0..255)
__device__ __forceinline__ bf16x8 deq8(uint32_t w0, uint32_t w1, float scale, float offset) {
    uint4 o;
    o.x = pack2(fmaf(scale, ubyte<0>(w0), -offset), fmaf(scale, ubyte<1>(w0), -offset));
    o.y = pack2(fmaf(scale, ubyte<2>(w0), -offset), fmaf(scale, ubyte<3>(w0), -offset));
    o.z = pack2(fmaf(scale, ubyte<0>(w1), -offset), fmaf(scale, ubyte<1>(w1), -offset));
    o.w = pack2(fmaf(scale, ubyte<2>(w1), -offset), fmaf(scale, ubyte<3>(w1), -offset));
    return __builtin_bit_cast(bf16x8, o);
}

// 6-bit scale and min of Q4_K sub-block j (0..7) from the header words hd.y, hd.z, hd.w (get_scale_min_k4)
__device__ __forceinline__ void k4_scale_min(uint4 hd, int j, float & sc, float & mn) {
    const int sh = 8 * (j & 3);
    if (j < 4) {
        sc = (float) ((hd.y >> sh) & 63u);
        mn = (float) ((hd.z >> sh) & 63u);
    } else {
        const uint32_t t = (hd.w >> sh) & 0xFFu;
        sc = (float) ((t & 0x0Fu) | ((((hd.y >> sh) >> 6) & 3u) << 4));
        mn = (float) ((t >> 4) | ((((hd.z >> sh) >> 6) & 3u) << 4));
    }
}

// R32 addressing of one weight row: group start g0, rows in the group rs, row inside it lr. Rows
// past M (a tile's tail, possibly whole groups past the end) read row M - 1 instead, so every load
// stays inside the tensor; their outputs are dropped.
struct RowAddr {
    int64_t g0;
    uint32_t rs, lr;
    __device__ RowAddr(int64_t M, int64_t m) {
        const int64_t mm = m < M ? m : M - 1;
        g0 = mm & ~(int64_t) 31;
        rs = (uint32_t) min<int64_t>(32, M - g0);
        lr = (uint32_t) (mm - g0);
    }
};

// ---- per format: one stage (128 elements of K) of one weight row for lane group g ---------------
// init() resolves the lane's row and lane group once (64-bit bases, 32-bit per-stage strides);
// load(s) fetches the lane's bytes of stage s into a Raw; prep() turns a Raw's block scales into
// the stage's fp32 factors; bop(raw, sc, t) is the lane's B fragment (8 bf16) for k-step t;
// chunk(g, t) is the 16-byte chunk (8 elements) of the stage's x row that the fragment pairs with.

template <int DT> struct PFmt;

// Q4_K: stage s = chunks 2 (s % 2), 2 (s % 2) + 1 of block s / 2; lane group g: unit 4 (s % 2) + g
// of the block (chunk c = 2 (s % 2) + g / 2, unit u = g % 2). k-step t: low (t < 2) / high nibbles
// of bytes 8 (t % 2) .. +7: elements 64c + 32 (t / 2) + 16u + 8 (t % 2) + e.
template <> struct PFmt<Q4_K> {
    struct Raw {
        uint4 q, hd;
    };
    struct Sc {
        float s0, o0, s1, o1;
    };
    const uint8_t * qb;
    const uint8_t * hb;
    uint32_t blk, half, hblk;
    int g;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb, const RowAddr & ra, int g_) {
        g = g_;
        qb = w + (uint64_t) ra.g0 * nb * 128 + (uint64_t) ra.lr * 16 + (uint64_t) g * ra.rs * 16;
        hb = w + (uint64_t) M * nb * 128 + (uint64_t) ra.g0 * nb * 16 + (uint64_t) ra.lr * 16;
        blk = ra.rs * 128;
        half = ra.rs * 64;
        hblk = ra.rs * 16;
    }
    __device__ Raw load(int64_t s) const {
        const uint32_t b = (uint32_t) (s >> 1), h = (uint32_t) (s & 1);
        return Raw{load16(qb + b * blk + h * half), load16(hb + b * hblk)};
    }
    __device__ Sc prep(const Raw & r, int64_t s) const {
        const int c = 2 * (int) (s & 1) + (g >> 1);
        const float d = half_bits(r.hd.x), dmin = half_bits(r.hd.x >> 16);
        float sc0, m0, sc1, m1;
        k4_scale_min(r.hd, 2 * c, sc0, m0);
        k4_scale_min(r.hd, 2 * c + 1, sc1, m1);
        return Sc{d * sc0, dmin * m0, d * sc1, dmin * m1};
    }
    __device__ static bf16x8 bop(const Raw & r, const Sc & c, int t) {
        const uint32_t w0 = (t & 1) ? r.q.z : r.q.x, w1 = (t & 1) ? r.q.w : r.q.y;
        const int sh = (t >> 1) * 4;
        return deq8((w0 >> sh) & 0x0F0F0F0Fu, (w1 >> sh) & 0x0F0F0F0Fu, t < 2 ? c.s0 : c.s1, t < 2 ? c.o0 : c.o1);
    }
    __device__ static int chunk(int g, int t) {
        return 8 * (g >> 1) + 4 * (t >> 1) + 2 * (g & 1) + (t & 1);
    }
};

// Q6_K: stage s = half h = s % 2 of block s / 2; lane group g: hf = g % 2 and runs
// rr = 2 (g / 2) + {0, 1} (units ql 4h + hf, ql 4h + 2 + hf, qh 8 + 2h + hf). k-step t: run
// rr = 2 (g / 2) + t / 2, elements 128h + 32rr + 16hf + 8 (t % 2) + e.
template <> struct PFmt<Q6_K> {
    struct Raw {
        uint4 qa, qc, qh, sc;
        uint32_t d;
    };
    struct Sc {
        float s0, s1;
    };
    const uint8_t * qb;
    const uint8_t * sb;
    const uint8_t * db;
    uint32_t blk, unit, sblk, dblk;
    int g;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb, const RowAddr & ra, int g_) {
        g = g_;
        qb = w + (uint64_t) ra.g0 * nb * 192 + (uint64_t) ra.lr * 16 + (uint64_t) (g & 1) * ra.rs * 16;
        sb = w + (uint64_t) M * nb * 192 + (uint64_t) ra.g0 * nb * 16 + (uint64_t) ra.lr * 16;
        db = w + (uint64_t) M * nb * 208 + (uint64_t) ra.g0 * nb * 2 + (uint64_t) ra.lr * 2;
        blk = ra.rs * 192;
        unit = ra.rs * 16;
        sblk = ra.rs * 16;
        dblk = ra.rs * 2;
    }
    __device__ Raw load(int64_t s) const {
        const uint32_t b = (uint32_t) (s >> 1), h = (uint32_t) (s & 1);
        const uint8_t * q = qb + b * blk;
        Raw r;
        r.qa = load16(q + (4 * h) * unit);     // ql[64h + 16hf + i]
        r.qc = load16(q + (4 * h + 2) * unit); // ql[64h + 32 + 16hf + i]
        r.qh = load16(q + (8 + 2 * h) * unit); // qh[32h + 16hf + i]
        r.sc = load16(sb + b * sblk);
        r.d = *reinterpret_cast<const uint16_t *>(db + b * dblk);
        return r;
    }
    // the signed 8-bit scales of the lane's two runs: bytes 8h + hf + 2rr (stored xor 0x80)
    __device__ Sc prep(const Raw & r, int64_t s) const {
        const int h = (int) (s & 1), hf = g & 1, rr = 2 * (g >> 1);
        const float d = half_bits(r.d);
        const int b0 = 8 * h + hf + 2 * rr, b1 = b0 + 2;
        const uint32_t w0 = b0 < 4 ? r.sc.x : b0 < 8 ? r.sc.y : b0 < 12 ? r.sc.z : r.sc.w;
        const uint32_t w1 = b1 < 4 ? r.sc.x : b1 < 8 ? r.sc.y : b1 < 12 ? r.sc.z : r.sc.w;
        return Sc{d * ((float) ((w0 >> (8 * (b0 & 3))) & 0xFFu) - 128.0f), d * ((float) ((w1 >> (8 * (b1 & 3))) & 0xFFu) - 128.0f)};
    }
    // 6-bit codes: low nibbles of qa (rr 0) / qc (rr 1), high nibbles (rr 2, 3), bits 2rr, 2rr + 1 of qh
    __device__ bf16x8 bop(const Raw & r, const Sc & c, int t) const {
        const int rr = 2 * (g >> 1) + (t >> 1);
        const uint4 ql = (t >> 1) ? r.qc : r.qa;
        const int ls = (g >> 1) * 4, hs = 2 * rr;
        const uint32_t l0 = (t & 1) ? ql.z : ql.x, l1 = (t & 1) ? ql.w : ql.y;
        const uint32_t h0 = (t & 1) ? r.qh.z : r.qh.x, h1 = (t & 1) ? r.qh.w : r.qh.y;
        const uint32_t v0 = ((l0 >> ls) & 0x0F0F0F0Fu) | (((h0 >> hs) << 4) & 0x30303030u);
        const uint32_t v1 = ((l1 >> ls) & 0x0F0F0F0Fu) | (((h1 >> hs) << 4) & 0x30303030u);
        const float ds = (t >> 1) ? c.s1 : c.s0;
        return deq8(v0, v1, ds, 32.0f * ds);
    }
    __device__ static int chunk(int g, int t) {
        return 4 * (2 * (g >> 1) + (t >> 1)) + 2 * (g & 1) + (t & 1);
    }
};

// Q8_0: stage s = blocks 4s .. 4s + 3; lane group g: block 4s + g (both units, d). k-step t: bytes
// 8t .. 8t + 7 = elements 32g + 8t + e. Blocks past the end of the row contribute zero.
template <> struct PFmt<Q8_0> {
    struct Raw {
        uint4 q0, q1;
        uint32_t d;
    };
    struct Sc {
        float s;
    };
    const uint8_t * qb;
    const uint8_t * db;
    uint32_t stage, unit, dstage;
    int64_t nb;
    int g;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb_, const RowAddr & ra, int g_) {
        g = g_;
        nb = nb_;
        qb = w + (uint64_t) ra.g0 * nb * 32 + (uint64_t) ra.lr * 16 + (uint64_t) g * ra.rs * 32;
        db = w + (uint64_t) M * nb * 32 + (uint64_t) ra.g0 * nb * 2 + (uint64_t) ra.lr * 2 + (uint64_t) g * ra.rs * 2;
        stage = ra.rs * 128;
        unit = ra.rs * 16;
        dstage = ra.rs * 8;
    }
    __device__ Raw load(int64_t s) const {
        const bool ok = s * 4 + g < nb;
        const uint32_t ss = ok ? (uint32_t) s : 0u; // past the row: a real block, scale 0
        Raw r;
        r.q0 = load16(qb + ss * stage);
        r.q1 = load16(qb + ss * stage + unit);
        r.d = ok ? *reinterpret_cast<const uint16_t *>(db + ss * dstage) : 0u;
        return r;
    }
    __device__ Sc prep(const Raw & r, int64_t) const {
        return Sc{half_bits(r.d)};
    }
    __device__ static bf16x8 bop(const Raw & r, const Sc & c, int t) {
        const uint4 & q = t < 2 ? r.q0 : r.q1;
        const uint32_t w0 = (t & 1) ? q.z : q.x, w1 = (t & 1) ? q.w : q.y;
        return deq8(w0, w1, c.s, 128.0f * c.s); // stored xor 0x80: value = (u - 128) * d
    }
    __device__ static int chunk(int g, int t) {
        return 4 * g + t;
    }
};

// Q4_0: stage s = blocks 4s .. 4s + 3; lane group g: block 4s + g. k-step t: low (t < 2) / high
// nibbles of bytes 8 (t % 2) .. +7 = elements 32g + 8t + e.
template <> struct PFmt<Q4_0> {
    struct Raw {
        uint4 q;
        uint32_t d;
    };
    struct Sc {
        float s;
    };
    const uint8_t * qb;
    const uint8_t * db;
    uint32_t stage, dstage;
    int64_t nb;
    int g;
    __device__ void init(const uint8_t * w, int64_t M, int64_t nb_, const RowAddr & ra, int g_) {
        g = g_;
        nb = nb_;
        qb = w + (uint64_t) ra.g0 * nb * 16 + (uint64_t) ra.lr * 16 + (uint64_t) g * ra.rs * 16;
        db = w + (uint64_t) M * nb * 16 + (uint64_t) ra.g0 * nb * 2 + (uint64_t) ra.lr * 2 + (uint64_t) g * ra.rs * 2;
        stage = ra.rs * 64;
        dstage = ra.rs * 8;
    }
    __device__ Raw load(int64_t s) const {
        const bool ok = s * 4 + g < nb;
        const uint32_t ss = ok ? (uint32_t) s : 0u;
        Raw r;
        r.q = load16(qb + ss * stage);
        r.d = ok ? *reinterpret_cast<const uint16_t *>(db + ss * dstage) : 0u;
        return r;
    }
    __device__ Sc prep(const Raw & r, int64_t) const {
        return Sc{half_bits(r.d)};
    }
    __device__ static bf16x8 bop(const Raw & r, const Sc & c, int t) {
        const uint32_t w0 = (t & 1) ? r.q.z : r.q.x, w1 = (t & 1) ? r.q.w : r.q.y;
        const int sh = (t >> 1) * 4;
        return deq8((w0 >> sh) & 0x0F0F0F0Fu, (w1 >> sh) & 0x0F0F0F0Fu, c.s, 8.0f * c.s);
    }
    __device__ static int chunk(int g, int t) {
        return 4 * g + t;
    }
};

struct MmArgs {
    MatArgs a;
    const uint16_t * xb; // bf16 activations [slices][N][K]
    float * part;        // split-K partial sums [split][slices][N][M] (split > 1)
    int64_t tiles_m, tiles_n;
    int64_t stages;      // stages of K (BK elements each)
    int split;           // work-groups along K per tile
};

// x tile in LDS: row n (token), 16-byte chunk c at (n * kChunks + (c ^ (n & 15))) * 8 bf16
__device__ __forceinline__ int xsw(int n, int c) {
    return (n * kChunks + (c ^ (n & 15))) * 8;
}

// the x tile of one stage: BN tokens x 16 chunks, BN / 16 chunks per thread (token p / 16, chunk
// p % 16 for p = threadIdx.x + 256 i); global pointers and LDS offsets resolved once
template <int BN>
struct XTile {
    static constexpr int NP = BN * kChunks / kThreads;
    const uint16_t * src[NP];
    int dst[NP];
    uint32_t kc[NP]; // element offset of the chunk inside a stage
    bool row_ok[NP];
    uint4 v[NP];
    __device__ void init(const uint16_t * xb, int64_t N, int64_t K, int64_t n0) {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int p = threadIdx.x + kThreads * i;
            const int64_t n = n0 + (p >> 4);
            row_ok[i] = n < N;
            kc[i] = 8 * (p & 15);
            src[i] = xb + (row_ok[i] ? n : 0) * K + kc[i];
            dst[i] = xsw(p >> 4, p & 15);
        }
    }
    // stage starting at element k0; `full` when all BK elements lie inside K
    __device__ void load(int64_t k0, int64_t K, bool full) {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const bool ok = row_ok[i] && (full || k0 + kc[i] < K);
            v[i] = ok ? *reinterpret_cast<const uint4 *>(src[i] + k0) : make_uint4(0, 0, 0, 0);
        }
    }
    __device__ void store(uint16_t * X) const {
#pragma unroll
        for (int i = 0; i < NP; ++i) *reinterpret_cast<uint4 *>(X + dst[i]) = v[i];
    }
};

template <int DT, int BN>
__global__ __launch_bounds__(kThreads, BN == 64 ? 3 : 2) void k_matmul(MmArgs L) {
    constexpr int NF = BN / 16; // token fragments per wave
    using F = PFmt<DT>;
    using Raw = typename F::Raw;
    extern __shared__ __attribute__((aligned(16))) uint16_t lds_mm[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int64_t tile = blockIdx.x / L.split;
    const int split = (int) (blockIdx.x % L.split);
    const int64_t tm = tile % L.tiles_m, tn = tile / L.tiles_m;
    const int64_t sl = blockIdx.y;
    const int64_t i2 = sl % L.a.ne12, i3 = sl / L.a.ne12;
    const uint8_t * w = L.a.w + (uint64_t) (i2 / L.a.r2) * L.a.w_s2 + (uint64_t) (i3 / L.a.r3) * L.a.w_s3;
    const int64_t K = L.a.K, N = L.a.N, M = L.a.M, nb = L.a.nb;
    const int64_t m0 = tm * BM, n0 = tn * BN;
    const int64_t s0 = L.stages * split / L.split, s1 = L.stages * (split + 1) / L.split;

    F f0, f1;
    f0.init(w, M, nb, RowAddr(M, m0 + 32 * wave + r), g);
    f1.init(w, M, nb, RowAddr(M, m0 + 32 * wave + 16 + r), g);
    XTile<BN> xt;
    xt.init(L.xb + (uint64_t) sl * N * K, N, K, n0);
    // LDS element offsets of the lane's A fragments: k-step t, token fragment f at aoff[t] + 16 f rows
    int aoff[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) aoff[t] = xsw(r, F::chunk(g, t));

    f32x4 acc[2][NF];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int f = 0; f < NF; ++f) acc[i][f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // one stage: MFMAs over the x tile in LDS buffer `buf` with the weights cw0 / cw1 (rows r,
    // r + 16 of the wave); meanwhile stage s + 1 is loaded into nw0 / nw1 and the x registers
    auto stage = [&](int64_t s, const Raw & cw0, const Raw & cw1, Raw & nw0, Raw & nw1) {
        const bool more = s + 1 < s1;
        if (more) {
            nw0 = f0.load(s + 1);
            nw1 = f1.load(s + 1);
            xt.load((s + 1) * BK, K, (s + 1) * BK + BK <= K);
        }
        const uint16_t * X = lds_mm + ((s - s0) & 1) * (BN * BK);
        const typename F::Sc sc0 = f0.prep(cw0, s), sc1 = f1.prep(cw1, s);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const bf16x8 b0 = f0.bop(cw0, sc0, t), b1 = f1.bop(cw1, sc1, t);
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                const bf16x8 a = *reinterpret_cast<const bf16x8 *>(X + aoff[t] + f * 16 * BK);
                acc[0][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b0, acc[0][f], 0, 0, 0);
                acc[1][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b1, acc[1][f], 0, 0, 0);
            }
        }
        if (more) xt.store(lds_mm + ((s + 1 - s0) & 1) * (BN * BK));
        __syncthreads();
    };
    Raw a0{}, a1{}, b0r{}, b1r{};
    if (s0 < s1) {
        a0 = f0.load(s0);
        a1 = f1.load(s0);
        xt.load(s0 * BK, K, s0 * BK + BK <= K);
        xt.store(lds_mm);
    }
    __syncthreads();
    for (int64_t s = s0; s < s1; s += 2) {
        stage(s, a0, a1, b0r, b1r);
        if (s + 1 < s1) stage(s + 1, b0r, b1r, a0, a1);
    }
    // acc[i][f], lane l: token 16 f + 4 (l / 16) + v, weight row 32 wave + 16 i + l % 16
    const int64_t slices = L.a.ne12 * L.a.ne13;
    float * y;
    int64_t ys1;
    if (L.split == 1) {
        y = L.a.y + i2 * L.a.y_s2 + i3 * L.a.y_s3;
        ys1 = L.a.y_s1;
    } else {
        y = L.part + ((uint64_t) split * slices + (uint64_t) sl) * N * M;
        ys1 = M;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t m = m0 + 32 * wave + 16 * i + r;
        if (m >= M) continue;
#pragma unroll
        for (int f = 0; f < NF; ++f) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t n = n0 + 16 * f + 4 * g + v;
                if (n < N) y[n * ys1 + m] = acc[i][f][v];
            }
        }
    }
}

// y = sum of the split-K partials, in split order. blockIdx.x is the row (token n of slice sl),
// blockIdx.y covers 1024 outputs of it; VEC when M and y's row starts allow float4 accesses.
template <bool VEC>
__global__ __launch_bounds__(256) void k_split_reduce(MmArgs L) {
    const int64_t N = L.a.N, M = L.a.M;
    const int64_t row = blockIdx.x, sl = row / N, n = row - sl * N;
    const int64_t i2 = sl % L.a.ne12, i3 = sl / L.a.ne12;
    const uint64_t plane = (uint64_t) L.a.ne12 * L.a.ne13 * N * M;
    const float * p = L.part + row * M;
    float * y = L.a.y + i2 * L.a.y_s2 + i3 * L.a.y_s3 + n * L.a.y_s1;
    const int64_t m = ((int64_t) blockIdx.y * 256 + threadIdx.x) * 4;
    if (VEC) {
        if (m >= M) return;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int sp = 0; sp < L.split; ++sp) {
            const float4 u = *reinterpret_cast<const float4 *>(p + sp * plane + m);
            v.x += u.x;
            v.y += u.y;
            v.z += u.z;
            v.w += u.w;
        }
        *reinterpret_cast<float4 *>(y + m) = v;
    } else {
        for (int64_t j = m; j < m + 4 && j < M; ++j) {
            float v = 0.0f;
            for (int sp = 0; sp < L.split; ++sp) v += p[sp * plane + j];
            y[j] = v;
        }
    }
}

// x (f32, strided rows) -> bf16 rows of K contiguous elements. blockIdx.x is the row (token n of
// slice sl), blockIdx.y covers 2048 elements of it; VEC when every row starts 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(256) void k_x_to_bf16(MatArgs a, uint16_t * xb) {
    const int64_t row = blockIdx.x, sl = row / a.N, n = row - sl * a.N;
    const int64_t i2 = sl % a.ne12, i3 = sl / a.ne12;
    const float * xp = a.x + i2 * a.x_s2 + i3 * a.x_s3 + n * a.x_s1;
    uint16_t * op = xb + row * a.K;
    const int64_t k = ((int64_t) blockIdx.y * 256 + threadIdx.x) * 8;
    if (k >= a.K) return; // K is a multiple of 32: a group of 8 lies inside the row or past it
    if (VEC) {
        const float4 u = *reinterpret_cast<const float4 *>(xp + k);
        const float4 v = *reinterpret_cast<const float4 *>(xp + k + 4);
        *reinterpret_cast<uint4 *>(op + k) = make_uint4(pack2(u.x, u.y), pack2(u.z, u.w), pack2(v.x, v.y), pack2(v.z, v.w));
    } else {
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = pack2(xp[k + 2 * j], xp[k + 2 * j + 1]);
        *reinterpret_cast<uint4 *>(op + k) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// Tile width and work-groups along K per tile. BN=64 runs three work-groups per CU, BN=128 two
// (the same MFMA rate per CU, half the dequantization per flop at BN=128). A problem with enough
// 64-wide tiles for three per CU takes BN=64 unsplit; otherwise BN=128 with enough splits for
// two work-groups per CU, each split keeping >= 8 stages of K.
struct MmConfig {
    int bn;
    int split;
};

MmConfig config_of(const MatArgs & a, int cu_count) {
    static const int env_bn = [] {
        const char * v = std::getenv("SCRAPGPU_HIP_MM_BN");
        return v != nullptr && *v ? (std::atoi(v) == 128 ? 128 : 64) : 0;
    }();
    static const int env_fill = [] {
        const char * v = std::getenv("SCRAPGPU_HIP_MM_FILL");
        return v != nullptr && *v ? std::max(1, std::atoi(v)) : 0;
    }();
    const int64_t slices = a.ne12 * a.ne13;
    const int64_t tm = (a.M + BM - 1) / BM;
    const int64_t stages = (a.K + BK - 1) / BK;
    auto tiles = [&](int bn) { return tm * ((a.N + bn - 1) / bn) * slices; };
    MmConfig c;
    c.bn = env_bn ? env_bn : (tiles(64) >= 3 * (int64_t) cu_count ? 64 : 128);
    const int64_t want = (int64_t) cu_count * (env_fill ? env_fill : (c.bn == 64 ? 3 : 2));
    static const int env_split = [] {
        const char * v = std::getenv("SCRAPGPU_HIP_MM_SPLIT");
        return v != nullptr && *v ? std::max(1, std::min(8, std::atoi(v))) : 0;
    }();
    c.split = 1;
    if (env_split) {
        c.split = (int) std::max<int64_t>(1, std::min<int64_t>(env_split, stages));
        return c;
    }
    while (tiles(c.bn) * c.split < want && stages / (c.split + 1) >= 8 && c.split < 8) ++c.split;
    return c;
}

size_t part_bytes(const MatArgs & a, int split) {
    return ((size_t) split * (size_t) (a.ne12 * a.ne13) * (size_t) a.N * (size_t) a.M * sizeof(float) + 255) / 256 * 256;
}

} // namespace

size_t matmul_scratch_bytes(const MatArgs & a, int cu_count) {
    const size_t xb = (size_t) a.N * (size_t) a.K * (size_t) (a.ne12 * a.ne13) * sizeof(uint16_t);
    const int split = config_of(a, cu_count).split;
    return split == 1 ? xb : (xb + 255) / 256 * 256 + part_bytes(a, split);
}

hipError_t launch_matmul_mfma(const MatArgs & a, uint8_t * scratch, int cu_count, hipStream_t stream, const char ** kernel_name) {
    const int64_t total = a.N * a.K * a.ne12 * a.ne13;
    uint16_t * xb = reinterpret_cast<uint16_t *>(scratch);
    const int64_t rows = a.N * a.ne12 * a.ne13;
    const bool vec = (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && a.x_s1 % 4 == 0 && a.x_s2 % 4 == 0 && a.x_s3 % 4 == 0;
    if (rows > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 cg((unsigned) rows, (unsigned) ((a.K + 2047) / 2048));
    if (vec)
        hipLaunchKernelGGL(k_x_to_bf16<true>, cg, dim3(256), 0, stream, a, xb);
    else
        hipLaunchKernelGGL(k_x_to_bf16<false>, cg, dim3(256), 0, stream, a, xb);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    MmArgs L;
    L.a = a;
    L.xb = xb;
    L.part = reinterpret_cast<float *>(scratch + ((size_t) total * sizeof(uint16_t) + 255) / 256 * 256);
    L.tiles_m = (a.M + BM - 1) / BM;
    const MmConfig cfg = config_of(a, cu_count);
    const int BN = cfg.bn;
    L.tiles_n = (a.N + BN - 1) / BN;
    L.stages = (a.K + BK - 1) / BK;
    L.split = cfg.split;
    const size_t lds = (size_t) 2 * BN * BK * sizeof(uint16_t);
    const int64_t slices = a.ne12 * a.ne13;
    const dim3 grid((unsigned) (L.tiles_m * L.tiles_n * L.split), (unsigned) slices);
    void * args[] = {&L};
    void * fn = nullptr;
    switch (a.dtype) {
        case Q4_0: fn = BN == 64 ? (void *) k_matmul<Q4_0, 64> : (void *) k_matmul<Q4_0, 128>; if (kernel_name) *kernel_name = "matmul_mfma_q4_0"; break;
        case Q8_0: fn = BN == 64 ? (void *) k_matmul<Q8_0, 64> : (void *) k_matmul<Q8_0, 128>; if (kernel_name) *kernel_name = "matmul_mfma_q8_0"; break;
        case Q4_K: fn = BN == 64 ? (void *) k_matmul<Q4_K, 64> : (void *) k_matmul<Q4_K, 128>; if (kernel_name) *kernel_name = "matmul_mfma_q4_k"; break;
        case Q6_K: fn = BN == 64 ? (void *) k_matmul<Q6_K, 64> : (void *) k_matmul<Q6_K, 128>; if (kernel_name) *kernel_name = "matmul_mfma_q6_k"; break;
        default: return hipErrorInvalidValue;
    }
    static bool attr_set = false; // LDS beyond the 64 KiB default (gfx950 has 160 KiB per CU)
    if (!attr_set) {
        for (void * f : {(void *) k_matmul<Q4_0, 128>, (void *) k_matmul<Q8_0, 128>, (void *) k_matmul<Q4_K, 128>, (void *) k_matmul<Q6_K, 128>}) {
            e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int) (2 * 128 * BK * sizeof(uint16_t)));
            if (e != hipSuccess) return e;
        }
        attr_set = true;
    }
    e = hipLaunchKernel(fn, grid, dim3(kThreads), args, lds, stream);
    if (e != hipSuccess || L.split == 1) return e;
    const bool yvec = (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 && a.M % 4 == 0 && a.y_s1 % 4 == 0 && a.y_s2 % 4 == 0 && a.y_s3 % 4 == 0;
    const dim3 rg((unsigned) rows, (unsigned) ((a.M + 1023) / 1024));
    if (yvec)
        hipLaunchKernelGGL(k_split_reduce<true>, rg, dim3(256), 0, stream, L);
    else
        hipLaunchKernelGGL(k_split_reduce<false>, rg, dim3(256), 0, stream, L);
    return hipGetLastError();
}

} // namespace sgk
