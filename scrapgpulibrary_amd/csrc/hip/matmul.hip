// Prefill matmul over R32 weights on the bf16 MFMA units of gfx950 (fp32 accumulate).
//
//   pre-pass   x (fp32, any column stride) -> xb (bf16, [N][K] contiguous) in stream scratch, once
//              per op, so that the GEMM reads half the activation bytes and never converts twice.
//   GEMM       a work-group (256 threads = 4 waves in 2 x 2) owns a BN x BM tile of y^T
//              (BN = 128 tokens x BM = 128 weight rows) over K in stages of BK = 64:
//                * the weights of the stage are loaded as 16-byte R32 units (coalesced), dequantized
//                  in registers (d*sc*q - dmin*m in fp32, rounded to bf16) and stored to LDS;
//                * the bf16 activations of the stage are copied to LDS;
//                * each wave runs v_mfma_f32_16x16x32_bf16 over its 64 x 64 sub-tile
//                  (A = activations, B = weights, so a lane's outputs are consecutive weight rows
//                  and the fp32 stores to y coalesce).
//              The global loads of a stage are issued P = 3 stages ahead into a register ring;
//              LDS is double-buffered (stage s + 1 is stored to the other buffer after the MFMAs
//              of stage s; one barrier per stage) and small enough (64 KB) for two work-groups per
//              CU. LDS rows are 128 bytes with XOR-swizzled 16-byte chunks: fragment reads and both
//              tile stores are free of bank conflicts.
#include "kernels.h"

#include <hip/hip_fp16.h>

#include <algorithm>

namespace sgk {
namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int P = 3; // stages in flight in registers
constexpr int LROW = BK; // bf16 per LDS row (128 bytes: 8 chunks of 16 bytes, XOR-swizzled)
constexpr int kThreads = 256;

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

// element offset of 16-byte chunk c (0..7) of LDS row r: chunks are XOR-swizzled with (r / 2) % 8 so
// that 16 consecutive rows at one chunk (MFMA fragment reads, weight stores) and 2 rows x 8 chunks
// (activation stores) each cover all 64 banks
__device__ __forceinline__ int sw(int r, int c) {
    return r * LROW + ((c ^ ((r >> 1) & 7)) << 3);
}

// 16 bf16 = scale * byte_i(q) - offset for the 16 bytes of q -> chunks c, c + 1 of row r
__device__ __forceinline__ void put16(uint16_t * T, int r, int c, uint4 q, float scale, float offset) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float b0 = (float) (w[i] & 0xFFu), b1 = (float) ((w[i] >> 8) & 0xFFu);
        const float b2 = (float) ((w[i] >> 16) & 0xFFu), b3 = (float) (w[i] >> 24);
        o[2 * i] = pack2(fmaf(scale, b0, -offset), fmaf(scale, b1, -offset));
        o[2 * i + 1] = pack2(fmaf(scale, b2, -offset), fmaf(scale, b3, -offset));
    }
    *reinterpret_cast<uint4 *>(T + sw(r, c)) = make_uint4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<uint4 *>(T + sw(r, c + 1)) = make_uint4(o[4], o[5], o[6], o[7]);
}

__device__ __forceinline__ uint4 mask4(uint4 q, uint32_t m) {
    return make_uint4(q.x & m, q.y & m, q.z & m, q.w & m);
}

__device__ __forceinline__ uint4 shr4(uint4 q, int s) {
    return make_uint4(q.x >> s, q.y >> s, q.z >> s, q.w >> s);
}

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

struct MmLaunch {
    MatArgs a;
    const uint16_t * xb;   // bf16 activations [slices][N][K]
    int64_t tiles_m, tiles_n;
};

// ---- weights: raw registers of one stage for one thread, and their dequantization to LDS ---------
// W tile layout in LDS: row m (0..BM-1) at W + m * LROW, k (0..BK-1) contiguous. A stage is BK = 64
// elements of K; thread t serves weight row t % 128 of the tile and half t / 128 of its stage work
// (a wave covers 64 consecutive rows: 512 contiguous bytes of every R32 unit it loads).

// per-thread R32 addressing of the thread's row: group start g0, rows in group rs, lane lr
struct RowAddr {
    int64_t g0;
    uint32_t rs, lr;
    bool live;
    __device__ RowAddr(int64_t M, int64_t m) {
        live = m < M;
        g0 = m & ~(int64_t) 31;
        rs = (uint32_t) min<int64_t>(32, M - g0);
        lr = (uint32_t) (m - g0);
    }
};

template <int DT> struct WStage;

// Q4_K: a stage is chunk c = (k0 % 256) / 64 of a block: units 2c (h = 0) and 2c + 1 (h = 1);
// thread: unit 2c + (t & 1) of its row (lo elements 16h + i, hi 32 + 16h + i) and the row header
template <> struct WStage<Q4_K> {
    uint4 q, hd;
    __device__ void load(const uint8_t * w, int64_t M, int64_t nb, const RowAddr & ra, int64_t k0) {
        if (!ra.live) return;
        const int64_t b = k0 >> 8;
        const int j = (int) ((k0 & 255) >> 5) + (threadIdx.x >> 7);
        q = load16(w + (uint64_t) ra.g0 * nb * 128 + (((uint64_t) b * 8 + j) * ra.rs + ra.lr) * 16);
        hd = load16(w + (uint64_t) M * nb * 128 + (uint64_t) ra.g0 * nb * 16 + ((uint64_t) b * ra.rs + ra.lr) * 16);
    }
    __device__ void store(uint16_t * W, const RowAddr & ra, int64_t k0, int64_t) const {
        const int row = threadIdx.x & 127, h = threadIdx.x >> 7;
        if (!ra.live) {
            put16(W, row, 2 * h, make_uint4(0, 0, 0, 0), 0.0f, 0.0f);
            put16(W, row, 4 + 2 * h, make_uint4(0, 0, 0, 0), 0.0f, 0.0f);
            return;
        }
        const int c = (int) ((k0 & 255) >> 6);
        const float d = half_bits(hd.x), dmin = half_bits(hd.x >> 16);
        float sc0, m0f, sc1, m1f;
        k4_scale_min(hd, 2 * c, sc0, m0f);
        k4_scale_min(hd, 2 * c + 1, sc1, m1f);
        put16(W, row, 2 * h, mask4(q, 0x0F0F0F0Fu), d * sc0, dmin * m0f);          // elements 16h + i
        put16(W, row, 4 + 2 * h, mask4(shr4(q, 4), 0x0F0F0F0Fu), d * sc1, dmin * m1f); // 32 + 16h + i
    }
};

// Q6_K: a stage is elements 64 rp .. 64 rp + 63 of half h of a block (r = 2 rp, 2 rp + 1); thread
// (row, hf): elements 32 (r - 2 rp) + 16 hf + i from units ql 4h+hf, ql 4h+2+hf, qh 8+2h+hf
template <> struct WStage<Q6_K> {
    uint4 qa, qc, qh, sc;
    uint32_t d;
    __device__ void load(const uint8_t * w, int64_t M, int64_t nb, const RowAddr & ra, int64_t k0) {
        if (!ra.live) return;
        const int hf = threadIdx.x >> 7;
        const int64_t b = k0 >> 8;
        const int h = (int) ((k0 & 255) >> 7);
        const uint8_t * qb = w + (uint64_t) ra.g0 * nb * 192 + ((uint64_t) b * 12 * ra.rs + ra.lr) * 16;
        qa = load16(qb + (uint64_t) (4 * h + hf) * ra.rs * 16);
        qc = load16(qb + (uint64_t) (4 * h + 2 + hf) * ra.rs * 16);
        qh = load16(qb + (uint64_t) (8 + 2 * h + hf) * ra.rs * 16);
        sc = load16(w + (uint64_t) M * nb * 192 + (uint64_t) ra.g0 * nb * 16 + ((uint64_t) b * ra.rs + ra.lr) * 16);
        d = *reinterpret_cast<const uint16_t *>(w + (uint64_t) M * nb * 208 + (uint64_t) ra.g0 * nb * 2 + ((uint64_t) b * ra.rs + ra.lr) * 2);
    }
    __device__ void store(uint16_t * W, const RowAddr & ra, int64_t k0, int64_t) const {
        const int row = threadIdx.x & 127, hf = threadIdx.x >> 7;
        if (!ra.live) {
            put16(W, row, 2 * hf, make_uint4(0, 0, 0, 0), 0.0f, 0.0f);
            put16(W, row, 4 + 2 * hf, make_uint4(0, 0, 0, 0), 0.0f, 0.0f);
            return;
        }
        const int h = (int) ((k0 & 255) >> 7), rp = (int) ((k0 & 127) >> 6);
        const float df = half_bits(d);
        uint4 v0, v1; // r = 2 rp and 2 rp + 1
        if (rp == 0) {
            v0 = make_uint4((qa.x & 0x0F0F0F0Fu) | ((qh.x << 4) & 0x30303030u), (qa.y & 0x0F0F0F0Fu) | ((qh.y << 4) & 0x30303030u),
                            (qa.z & 0x0F0F0F0Fu) | ((qh.z << 4) & 0x30303030u), (qa.w & 0x0F0F0F0Fu) | ((qh.w << 4) & 0x30303030u));
            v1 = make_uint4((qc.x & 0x0F0F0F0Fu) | ((qh.x << 2) & 0x30303030u), (qc.y & 0x0F0F0F0Fu) | ((qh.y << 2) & 0x30303030u),
                            (qc.z & 0x0F0F0F0Fu) | ((qh.z << 2) & 0x30303030u), (qc.w & 0x0F0F0F0Fu) | ((qh.w << 2) & 0x30303030u));
        } else {
            v0 = make_uint4(((qa.x >> 4) & 0x0F0F0F0Fu) | (qh.x & 0x30303030u), ((qa.y >> 4) & 0x0F0F0F0Fu) | (qh.y & 0x30303030u),
                            ((qa.z >> 4) & 0x0F0F0F0Fu) | (qh.z & 0x30303030u), ((qa.w >> 4) & 0x0F0F0F0Fu) | (qh.w & 0x30303030u));
            v1 = make_uint4(((qc.x >> 4) & 0x0F0F0F0Fu) | ((qh.x >> 2) & 0x30303030u), ((qc.y >> 4) & 0x0F0F0F0Fu) | ((qh.y >> 2) & 0x30303030u),
                            ((qc.z >> 4) & 0x0F0F0F0Fu) | ((qh.z >> 2) & 0x30303030u), ((qc.w >> 4) & 0x0F0F0F0Fu) | ((qh.w >> 2) & 0x30303030u));
        }
        // scale bytes 8h + 2r + hf (stored xor 0x80), r = 2 rp, 2 rp + 1: word 2h + rp, bytes hf, 2 + hf
        const uint32_t sw = h ? (rp ? sc.w : sc.z) : (rp ? sc.y : sc.x);
        const float ds0 = df * (float) (int8_t) (((sw >> (8 * hf)) & 0xFFu) ^ 0x80u);
        const float ds1 = df * (float) (int8_t) (((sw >> (8 * (2 + hf))) & 0xFFu) ^ 0x80u);
        put16(W, row, 2 * hf, v0, ds0, 32.0f * ds0);     // elements 16hf + i
        put16(W, row, 4 + 2 * hf, v1, ds1, 32.0f * ds1); // 32 + 16hf + i
    }
};

// Q8_0: a stage is 2 blocks; thread: block (k0 / 32) + (t & 1) of its row, both units
template <> struct WStage<Q8_0> {
    uint4 q0, q1;
    uint32_t d;
    __device__ void load(const uint8_t * w, int64_t M, int64_t nb, const RowAddr & ra, int64_t k0) {
        const int64_t b = (k0 >> 5) + (threadIdx.x >> 7);
        if (!ra.live || b >= nb) return;
        q0 = load16(w + (uint64_t) ra.g0 * nb * 32 + (((uint64_t) b * 2) * ra.rs + ra.lr) * 16);
        q1 = load16(w + (uint64_t) ra.g0 * nb * 32 + (((uint64_t) b * 2 + 1) * ra.rs + ra.lr) * 16);
        d = *reinterpret_cast<const uint16_t *>(w + (uint64_t) M * nb * 32 + (uint64_t) ra.g0 * nb * 2 + ((uint64_t) b * ra.rs + ra.lr) * 2);
    }
    __device__ void store(uint16_t * W, const RowAddr & ra, int64_t k0, int64_t nb) const {
        const int row = threadIdx.x & 127, half = threadIdx.x >> 7;
        const bool ok = ra.live && (k0 >> 5) + half < nb;
        const float df = ok ? half_bits(d) : 0.0f;
        const uint4 z = make_uint4(0, 0, 0, 0);
        put16(W, row, 4 * half, ok ? q0 : z, df, 128.0f * df); // stored xor 0x80: value = (u - 128) * d
        put16(W, row, 4 * half + 2, ok ? q1 : z, df, 128.0f * df);
    }
};

// Q4_0: a stage is 2 blocks; thread: block (k0 / 32) + (t & 1) of its row
template <> struct WStage<Q4_0> {
    uint4 q;
    uint32_t d;
    __device__ void load(const uint8_t * w, int64_t M, int64_t nb, const RowAddr & ra, int64_t k0) {
        const int64_t b = (k0 >> 5) + (threadIdx.x >> 7);
        if (!ra.live || b >= nb) return;
        q = load16(w + (uint64_t) ra.g0 * nb * 16 + ((uint64_t) b * ra.rs + ra.lr) * 16);
        d = *reinterpret_cast<const uint16_t *>(w + (uint64_t) M * nb * 16 + (uint64_t) ra.g0 * nb * 2 + ((uint64_t) b * ra.rs + ra.lr) * 2);
    }
    __device__ void store(uint16_t * W, const RowAddr & ra, int64_t k0, int64_t nb) const {
        const int row = threadIdx.x & 127, half = threadIdx.x >> 7;
        const bool ok = ra.live && (k0 >> 5) + half < nb;
        const float df = ok ? half_bits(d) : 0.0f;
        const uint4 q0 = ok ? q : make_uint4(0, 0, 0, 0);
        put16(W, row, 4 * half, mask4(q0, 0x0F0F0F0Fu), df, 8.0f * df);
        put16(W, row, 4 * half + 2, mask4(shr4(q0, 4), 0x0F0F0F0Fu), df, 8.0f * df);
    }
};

// ---- activations: BN tokens x BK k of bf16 = 1024 16-byte pieces -> 4 per thread ---------------
struct XStage {
    uint4 v[4];
    __device__ void load(const uint16_t * xb, int64_t N, int64_t K, int64_t n0, int64_t k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = threadIdx.x + kThreads * i; // piece: row p / 8, k 8 (p % 8)
            const int64_t n = n0 + (p >> 3), k = k0 + 8 * (p & 7);
            v[i] = n < N && k < K ? *reinterpret_cast<const uint4 *>(xb + n * K + k) : make_uint4(0, 0, 0, 0);
        }
    }
    __device__ void store(uint16_t * X) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = threadIdx.x + kThreads * i;
            *reinterpret_cast<uint4 *>(X + sw(p >> 3, p & 7)) = v[i];
        }
    }
};

template <int DT>
__global__ __launch_bounds__(kThreads, 2) void k_matmul(MmLaunch L) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds_mm[];
    // LDS buffer b: weights at lds_mm + b * (BM + BN) * LROW, activations BM rows further
    auto Wbuf = [&](int b) { return lds_mm + b * (BM + BN) * LROW; };
    auto Xbuf = [&](int b) { return lds_mm + b * (BM + BN) * LROW + BM * LROW; };
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1; // wave tile: tokens 64 wn.., weight rows 64 wm..
    const int64_t tm = blockIdx.x % L.tiles_m, tn = blockIdx.x / L.tiles_m;
    const int64_t sl = blockIdx.y;
    const int64_t i2 = sl % L.a.ne12, i3 = sl / L.a.ne12;
    const uint8_t * w = L.a.w + (uint64_t) (i2 / L.a.r2) * L.a.w_s2 + (uint64_t) (i3 / L.a.r3) * L.a.w_s3;
    const int64_t K = L.a.K, N = L.a.N, M = L.a.M, nb = L.a.nb;
    const uint16_t * xb = L.xb + (uint64_t) sl * N * K;
    float * y = L.a.y + i2 * L.a.y_s2 + i3 * L.a.y_s3;
    const int64_t m0 = tm * BM, n0 = tn * BN;
    const int stages = (int) ((K + BK - 1) / BK);
    const RowAddr ra(M, m0 + (tid & 127));

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // register ring: slot s % P holds stage s from its load until its store to LDS
    WStage<DT> ws[P];
    XStage xs[P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        if (j < stages) {
            ws[j].load(w, M, nb, ra, (int64_t) j * BK);
            xs[j].load(xb, N, K, n0, (int64_t) j * BK);
        }
    }
    ws[0].store(Wbuf(0), ra, 0, nb);
    xs[0].store(Xbuf(0));
    if (P < stages) {
        ws[0].load(w, M, nb, ra, (int64_t) P * BK);
        xs[0].load(xb, N, K, n0, (int64_t) P * BK);
    }
    __syncthreads();

    for (int s0 = 0; s0 < stages; s0 += P) {
#pragma unroll
        for (int j = 0; j < P; ++j) {
            const int s = s0 + j;
            if (s < stages) {
                const uint16_t * Xc = Xbuf(s & 1);
                const uint16_t * Wc = Wbuf(s & 1);
#pragma unroll
                for (int kk = 0; kk < BK; kk += 32) {
                    bf16x8 af[4], bfr[4];
                    const int cq = (kk >> 3) + (lane >> 4); // 16-byte chunk of the lane's 8 k values
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        af[i] = *reinterpret_cast<const bf16x8 *>(Xc + sw(64 * wn + 16 * i + (lane & 15), cq));
                        bfr[i] = *reinterpret_cast<const bf16x8 *>(Wc + sw(64 * wm + 16 * i + (lane & 15), cq));
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int jj = 0; jj < 4; ++jj)
                            acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[jj], acc[i][jj], 0, 0, 0);
                }
                // stage s + 1 (ring slot (j + 1) % P) goes to the other LDS buffer; the slot then
                // receives stage s + 1 + P
                const int nj = (j + 1) % P;
                if (s + 1 < stages) {
                    ws[nj].store(Wbuf((s + 1) & 1), ra, (int64_t) (s + 1) * BK, nb);
                    xs[nj].store(Xbuf((s + 1) & 1));
                    if (s + 1 + P < stages) {
                        ws[nj].load(w, M, nb, ra, (int64_t) (s + 1 + P) * BK);
                        xs[nj].load(xb, N, K, n0, (int64_t) (s + 1 + P) * BK);
                    }
                }
                __syncthreads();
            }
        }
    }
    // acc[i][j], lane l: token 64 wn + 16 i + 4 (l / 16) + r, weight row 64 wm + 16 j + l % 16
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t n = n0 + 64 * wn + 16 * i + 4 * (lane >> 4) + r;
            if (n >= N) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t m = m0 + 64 * wm + 16 * j + (lane & 15);
                if (m < M) y[n * L.a.y_s1 + m] = acc[i][j][r];
            }
        }
    }
}

// x (fp32, strided) -> xb (bf16, [slice][N][K] contiguous)
__global__ __launch_bounds__(256) void k_x_to_bf16(MatArgs a, uint16_t * xb) {
    const int64_t per = a.N * a.K;
    const int64_t total = per * a.ne12 * a.ne13;
    for (int64_t i = ((int64_t) blockIdx.x * blockDim.x + threadIdx.x) * 2; i < total; i += (int64_t) gridDim.x * blockDim.x * 2) {
        const int64_t sl = i / per, rem = i - sl * per;
        const int64_t n = rem / a.K, k = rem - n * a.K; // K is even: the pair stays in one row
        const int64_t i2 = sl % a.ne12, i3 = sl / a.ne12;
        const float * xp = a.x + i2 * a.x_s2 + i3 * a.x_s3 + n * a.x_s1 + k;
        *reinterpret_cast<uint32_t *>(xb + i) = pack2(xp[0], xp[1]);
    }
}

} // namespace

size_t matmul_scratch_bytes(const MatArgs & a) {
    return (size_t) a.N * (size_t) a.K * (size_t) (a.ne12 * a.ne13) * sizeof(uint16_t);
}

hipError_t launch_matmul_mfma(const MatArgs & a, uint16_t * scratch, int cu_count, hipStream_t stream, const char ** kernel_name) {
    (void) cu_count;
    const int64_t total = a.N * a.K * a.ne12 * a.ne13;
    const unsigned pg = (unsigned) std::min<int64_t>(std::max<int64_t>(1, (total / 2 + 255) / 256), 8192);
    hipLaunchKernelGGL(k_x_to_bf16, dim3(pg), dim3(256), 0, stream, a, scratch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    MmLaunch L;
    L.a = a;
    L.xb = scratch;
    L.tiles_m = (a.M + BM - 1) / BM;
    L.tiles_n = (a.N + BN - 1) / BN;
    const size_t lds = (size_t) 2 * (BM + BN) * LROW * sizeof(uint16_t);
    const dim3 grid((unsigned) (L.tiles_m * L.tiles_n), (unsigned) (a.ne12 * a.ne13));
    void * args[] = {&L};
    void * fn = nullptr;
    switch (a.dtype) {
        case Q4_0: fn = (void *) k_matmul<Q4_0>; if (kernel_name) *kernel_name = "matmul_mfma_q4_0"; break;
        case Q8_0: fn = (void *) k_matmul<Q8_0>; if (kernel_name) *kernel_name = "matmul_mfma_q8_0"; break;
        case Q4_K: fn = (void *) k_matmul<Q4_K>; if (kernel_name) *kernel_name = "matmul_mfma_q4_k"; break;
        case Q6_K: fn = (void *) k_matmul<Q6_K>; if (kernel_name) *kernel_name = "matmul_mfma_q6_k"; break;
        default: return hipErrorInvalidValue;
    }
    static bool attr_set = false; // LDS beyond the 64 KiB default (gfx950 has 160 KiB per CU)
    if (!attr_set) {
        for (void * f : {(void *) k_matmul<Q4_0>, (void *) k_matmul<Q8_0>, (void *) k_matmul<Q4_K>, (void *) k_matmul<Q6_K>}) {
            e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
            if (e != hipSuccess) return e;
        }
        attr_set = true;
    }
    return hipLaunchKernel(fn, grid, dim3(kThreads), args, lds, stream);
}

} // namespace sgk
