// Prefill matmul over R32 weights on the bf16 MFMA units of gfx950 (fp32 accumulate).
//
// A work-group (256 threads, 4 waves in a 2 x 2 arrangement) computes a BM x BN tile of y^T
// (BM output rows of W, BN columns of x) over K in steps of BK = 256 elements:
//   1. the BM x BK weights are dequantized from R32 (coalesced 16-byte units, scales decoded per
//      unit) to bf16 in LDS, rounding d*sc*q - dmin*m computed in fp32;
//   2. the BN x BK activations are converted fp32 -> bf16 into LDS;
//   3. each wave runs v_mfma_f32_16x16x32_bf16 over its 64 x 64 sub-tile (4 x 4 MFMA tiles).
// LDS rows are padded by 16 bytes so that the 16 lanes reading 16 rows of one k-slice hit
// different banks.
#include "kernels.h"

#include <hip/hip_fp16.h>

#include <algorithm>

namespace sgk {
namespace {

constexpr int BM = 128, BN = 128, BK = 256;
constexpr int LDSROW = BK + 8; // bf16 elements per LDS row (16 bytes of padding)
constexpr int kThreads = 256;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint16_t to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u); // round to nearest even (inputs are finite)
    return (uint16_t) (u >> 16);
}

__device__ __forceinline__ float half_bits(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short) (h & 0xFFFFu)));
}

__device__ __forceinline__ uint4 load16(const uint8_t * p) {
    return *reinterpret_cast<const uint4 *>(p);
}

__device__ __forceinline__ uint32_t byte_of(uint4 v, int i) {
    const uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return (w >> (8 * (i & 3))) & 0xFFu;
}

// writes 16 bf16 values v[i] = scale * byte_i - offset at dst[0..15]
__device__ __forceinline__ void put16(uint16_t * dst, uint4 q, float scale, float offset) {
    uint32_t out[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float a = scale * (float) byte_of(q, 2 * i) - offset;
        const float b = scale * (float) byte_of(q, 2 * i + 1) - offset;
        out[i] = (uint32_t) to_bf16(a) | ((uint32_t) to_bf16(b) << 16);
    }
    uint4 * d = reinterpret_cast<uint4 *>(dst);
    d[0] = make_uint4(out[0], out[1], out[2], out[3]);
    d[1] = make_uint4(out[4], out[5], out[6], out[7]);
}

__device__ __forceinline__ uint4 mask4(uint4 q, uint32_t m) {
    return make_uint4(q.x & m, q.y & m, q.z & m, q.w & m);
}

__device__ __forceinline__ uint4 shr4(uint4 q, int s) {
    return make_uint4(q.x >> s, q.y >> s, q.z >> s, q.w >> s);
}

struct MmLaunch {
    MatArgs a;
    int64_t tiles_m, tiles_n;
};

// dequantize the weights of rows [m0, m0 + BM) x k [k0, k0 + BK) into W (zeros outside the matrix)
template <int DT>
__device__ void stage_w(const MmLaunch & L, const uint8_t * w, int64_t m0, int64_t k0, uint16_t * W) {
    const int tid = threadIdx.x;
    const int64_t M = L.a.M, nb = L.a.nb;
    if (DT == Q4_K || DT == Q6_K) {
        const int64_t b = k0 / 256;
        if (DT == Q4_K) {
            // 4 groups x 8 units x 32 rows
            for (int u = tid; u < 4 * 8 * 32; u += kThreads) {
                const int gq = u >> 8, j = (u >> 5) & 7, row = u & 31;
                const int64_t g0 = m0 + 32 * gq;
                uint16_t * dst = W + (32 * gq + row) * LDSROW;
                const int c = j >> 1, h = j & 1;
                if (g0 + row >= M) {
                    put16(dst + 64 * c + 16 * h, make_uint4(0, 0, 0, 0), 0.0f, 0.0f);
                    put16(dst + 64 * c + 32 + 16 * h, make_uint4(0, 0, 0, 0), 0.0f, 0.0f);
                    continue;
                }
                const int rs = (int) min<int64_t>(32, M - g0);
                const uint4 q = load16(w + (uint64_t) g0 * nb * 128 + (((uint64_t) b * 8 + j) * rs + row) * 16);
                const uint4 hd = load16(w + (uint64_t) M * nb * 128 + (uint64_t) g0 * nb * 16 + ((uint64_t) b * rs + row) * 16);
                const float d = half_bits(hd.x), dmin = half_bits(hd.x >> 16);
                const uint4 sv = make_uint4(hd.y, hd.z, hd.w, 0u);
                uint32_t sc[2], mn[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int jj = 2 * c + t;
                    if (jj < 4) {
                        sc[t] = byte_of(sv, jj) & 63u;
                        mn[t] = byte_of(sv, jj + 4) & 63u;
                    } else {
                        sc[t] = (byte_of(sv, jj + 4) & 0x0Fu) | ((byte_of(sv, jj - 4) >> 6) << 4);
                        mn[t] = (byte_of(sv, jj + 4) >> 4) | ((byte_of(sv, jj) >> 6) << 4);
                    }
                }
                put16(dst + 64 * c + 16 * h, mask4(q, 0x0F0F0F0Fu), d * (float) sc[0], dmin * (float) mn[0]);
                put16(dst + 64 * c + 32 + 16 * h, mask4(shr4(q, 4), 0x0F0F0F0Fu), d * (float) sc[1], dmin * (float) mn[1]);
            }
        } else {
            // 4 groups x 4 tasks (h, l16) x 32 rows; a task covers 64 elements
            for (int u = tid; u < 4 * 4 * 32; u += kThreads) {
                const int gq = u >> 7, task = (u >> 5) & 3, row = u & 31;
                const int h = task >> 1, hf = task & 1;
                const int64_t g0 = m0 + 32 * gq;
                uint16_t * dst = W + (32 * gq + row) * LDSROW + 128 * h + 16 * hf;
                if (g0 + row >= M) {
                    for (int r = 0; r < 4; ++r) put16(dst + 32 * r, make_uint4(0, 0, 0, 0), 0.0f, 0.0f);
                    continue;
                }
                const int rs = (int) min<int64_t>(32, M - g0);
                const uint8_t * qb = w + (uint64_t) g0 * nb * 192 + ((uint64_t) b * 12 * rs + row) * 16;
                const uint4 qa = load16(qb + (uint64_t) (4 * h + hf) * rs * 16);
                const uint4 qc = load16(qb + (uint64_t) (4 * h + 2 + hf) * rs * 16);
                const uint4 qh = load16(qb + (uint64_t) (8 + 2 * h + hf) * rs * 16);
                const uint4 scv = load16(w + (uint64_t) M * nb * 192 + (uint64_t) g0 * nb * 16 + ((uint64_t) b * rs + row) * 16);
                const float d = half_bits(*reinterpret_cast<const uint16_t *>(w + (uint64_t) M * nb * 208 + (uint64_t) g0 * nb * 2 + ((uint64_t) b * rs + row) * 2));
                const uint4 v0 = make_uint4((qa.x & 0x0F0F0F0Fu) | ((qh.x << 4) & 0x30303030u), (qa.y & 0x0F0F0F0Fu) | ((qh.y << 4) & 0x30303030u),
                                            (qa.z & 0x0F0F0F0Fu) | ((qh.z << 4) & 0x30303030u), (qa.w & 0x0F0F0F0Fu) | ((qh.w << 4) & 0x30303030u));
                const uint4 v1 = make_uint4((qc.x & 0x0F0F0F0Fu) | ((qh.x << 2) & 0x30303030u), (qc.y & 0x0F0F0F0Fu) | ((qh.y << 2) & 0x30303030u),
                                            (qc.z & 0x0F0F0F0Fu) | ((qh.z << 2) & 0x30303030u), (qc.w & 0x0F0F0F0Fu) | ((qh.w << 2) & 0x30303030u));
                const uint4 v2 = make_uint4(((qa.x >> 4) & 0x0F0F0F0Fu) | (qh.x & 0x30303030u), ((qa.y >> 4) & 0x0F0F0F0Fu) | (qh.y & 0x30303030u),
                                            ((qa.z >> 4) & 0x0F0F0F0Fu) | (qh.z & 0x30303030u), ((qa.w >> 4) & 0x0F0F0F0Fu) | (qh.w & 0x30303030u));
                const uint4 v3 = make_uint4(((qc.x >> 4) & 0x0F0F0F0Fu) | ((qh.x >> 2) & 0x30303030u), ((qc.y >> 4) & 0x0F0F0F0Fu) | ((qh.y >> 2) & 0x30303030u),
                                            ((qc.z >> 4) & 0x0F0F0F0Fu) | ((qh.z >> 2) & 0x30303030u), ((qc.w >> 4) & 0x0F0F0F0Fu) | ((qh.w >> 2) & 0x30303030u));
                const uint4 vv[4] = {v0, v1, v2, v3};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float ds = d * (float) (int8_t) (byte_of(scv, 8 * h + 2 * r + hf) ^ 0x80u);
                    put16(dst + 32 * r, vv[r], ds, 32.0f * ds);
                }
            }
        }
        return;
    }
    // Q4_0 / Q8_0: BK covers up to 8 blocks of 32
    const int64_t b0 = k0 / 32;
    const int nblk = (int) min<int64_t>(8, nb - b0);
    if (DT == Q4_0) {
        for (int u = tid; u < 128 * 8; u += kThreads) {
            const int row = u >> 3, bi = u & 7; // one unit per (row, block)
            const int64_t m = m0 + row;
            uint16_t * dst = W + row * LDSROW + 32 * bi;
            if (m >= M || bi >= nblk) {
                put16(dst, make_uint4(0, 0, 0, 0), 0.0f, 0.0f);
                put16(dst + 16, make_uint4(0, 0, 0, 0), 0.0f, 0.0f);
                continue;
            }
            const int64_t g0 = m - (m & 31);
            const int lane = (int) (m & 31);
            const int rs = (int) min<int64_t>(32, M - g0);
            const int64_t b = b0 + bi;
            const uint4 q = load16(w + (uint64_t) g0 * nb * 16 + ((uint64_t) b * rs + lane) * 16);
            const float d = half_bits(*reinterpret_cast<const uint16_t *>(w + (uint64_t) M * nb * 16 + (uint64_t) g0 * nb * 2 + ((uint64_t) b * rs + lane) * 2));
            put16(dst, mask4(q, 0x0F0F0F0Fu), d, 8.0f * d);
            put16(dst + 16, mask4(shr4(q, 4), 0x0F0F0F0Fu), d, 8.0f * d);
        }
    } else {
        for (int u = tid; u < 128 * 16; u += kThreads) {
            const int row = u >> 4, bi = (u >> 1) & 7, hf = u & 1;
            const int64_t m = m0 + row;
            uint16_t * dst = W + row * LDSROW + 32 * bi + 16 * hf;
            if (m >= M || bi >= nblk) {
                put16(dst, make_uint4(0, 0, 0, 0), 0.0f, 0.0f);
                continue;
            }
            const int64_t g0 = m - (m & 31);
            const int lane = (int) (m & 31);
            const int rs = (int) min<int64_t>(32, M - g0);
            const int64_t b = b0 + bi;
            const uint4 u8 = load16(w + (uint64_t) g0 * nb * 32 + (((uint64_t) b * 2 + hf) * rs + lane) * 16);
            const float d = half_bits(*reinterpret_cast<const uint16_t *>(w + (uint64_t) M * nb * 32 + (uint64_t) g0 * nb * 2 + ((uint64_t) b * rs + lane) * 2));
            put16(dst, u8, d, 128.0f * d); // stored xor 0x80: value = (u - 128) * d
        }
    }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void k_matmul(MmLaunch L) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds_mm[];
    uint16_t * W = lds_mm;
    uint16_t * X = lds_mm + BM * LDSROW;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int64_t tm = blockIdx.x % L.tiles_m, tn = blockIdx.x / L.tiles_m;
    const int64_t sl = blockIdx.y;
    const int64_t i2 = sl % L.a.ne12, i3 = sl / L.a.ne12;
    const uint8_t * w = L.a.w + (uint64_t) (i2 / L.a.r2) * L.a.w_s2 + (uint64_t) (i3 / L.a.r3) * L.a.w_s3;
    const float * x = L.a.x + i2 * L.a.x_s2 + i3 * L.a.x_s3;
    float * y = L.a.y + i2 * L.a.y_s2 + i3 * L.a.y_s3;
    const int64_t m0 = tm * BM, n0 = tn * BN;
    const int64_t K = L.a.K, N = L.a.N;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int64_t k0 = 0; k0 < K; k0 += BK) {
        stage_w<DT>(L, w, m0, k0, W);
        const int kl = (int) min<int64_t>(BK, K - k0);
        for (int i = tid; i < BN * BK; i += kThreads) {
            const int n = i / BK, k = i % BK;
            const float v = (n0 + n < N && k < kl) ? x[(n0 + n) * L.a.x_s1 + k0 + k] : 0.0f;
            X[n * LDSROW + k] = to_bf16(v);
        }
        __syncthreads();
#pragma unroll 2
        for (int kk = 0; kk < BK; kk += 32) {
            bf16x8 af[4], bfr[4];
            const int kq = kk + 8 * (lane >> 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                af[i] = *reinterpret_cast<const bf16x8 *>(W + (64 * wm + 16 * i + (lane & 15)) * LDSROW + kq);
                bfr[i] = *reinterpret_cast<const bf16x8 *>(X + (64 * wn + 16 * i + (lane & 15)) * LDSROW + kq);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    // acc[i][j] lane l: rows (of W) 16i + 4(l/16) + r, column (of x) 16j + l%16
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t n = n0 + 64 * wn + 16 * j + (lane & 15);
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + 64 * wm + 16 * i + 4 * (lane >> 4) + r;
                if (m < L.a.M) y[n * L.a.y_s1 + m] = acc[i][j][r];
            }
        }
    }
}

} // namespace

hipError_t launch_matmul_mfma(const MatArgs & a, int cu_count, hipStream_t stream, const char ** kernel_name) {
    (void) cu_count;
    MmLaunch L;
    L.a = a;
    L.tiles_m = (a.M + BM - 1) / BM;
    L.tiles_n = (a.N + BN - 1) / BN;
    const size_t lds = (size_t) (BM + BN) * LDSROW * sizeof(uint16_t);
    const dim3 grid((unsigned) (L.tiles_m * L.tiles_n), (unsigned) (a.ne12 * a.ne13));
    void * args[] = {&L};
    void * fn = nullptr;
    static bool attr_set = false; // LDS beyond the 64 KiB default (gfx950 has 160 KiB per CU)
    switch (a.dtype) {
        case Q4_0: fn = (void *) k_matmul<Q4_0>; if (kernel_name) *kernel_name = "matmul_mfma_q4_0"; break;
        case Q8_0: fn = (void *) k_matmul<Q8_0>; if (kernel_name) *kernel_name = "matmul_mfma_q8_0"; break;
        case Q4_K: fn = (void *) k_matmul<Q4_K>; if (kernel_name) *kernel_name = "matmul_mfma_q4_k"; break;
        case Q6_K: fn = (void *) k_matmul<Q6_K>; if (kernel_name) *kernel_name = "matmul_mfma_q6_k"; break;
        default: return hipErrorInvalidValue;
    }
    if (!attr_set) {
        for (void * f : {(void *) k_matmul<Q4_0>, (void *) k_matmul<Q8_0>, (void *) k_matmul<Q4_K>, (void *) k_matmul<Q6_K>}) {
            const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
            if (e != hipSuccess) return e;
        }
        attr_set = true;
    }
    return hipLaunchKernel(fn, grid, dim3(kThreads), args, lds, stream);
}

} // namespace sgk
