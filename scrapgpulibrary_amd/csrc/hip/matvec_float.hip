// Decode matvec over float weights (F32 / F16 / BF16 rows in the natural layout) for 1 <= N <= 8
// columns (gfx950, wave64).
//
// Replaces, for the hip backend, the reference's float-weight matvec kernels (the F32 / F16 arms
// of src/backends/opencl11/ops_matmul.cpp:67-123, kernels/mul_mv.cl) with the product of the CPU
// reference's exec_mul_mat (src/core/ref/ops.cpp:891-984): y[n, m] = sum_k W[m, k] x[n, k], every
// weight widened exactly to f32 (F16 through the hardware conversion, BF16 as the high half of an
// f32) and multiplied by f32 x in f32. Only the summation order differs from the reference
// (per-lane partial sums of 8 consecutive elements, then a tree), a difference of ~K 2^-24 of the
// products' magnitudes.
//
// Work decomposition: a work-group of 4 waves owns 8 rows and all of K. K is dealt in steps of 512
// elements (8 per lane, one 16- or 32-byte load per row); wave w takes steps w, w + 4, ..., two at
// a time with every load of both issued before any arithmetic. At the end each wave folds its 64
// lanes' partial sums with a reduce-scatter butterfly (8 N values per lane -> one value per lane in
// 8 N - 1 + log2(64 / 8 N) exchanges instead of 6 per value), and the 4 waves meet in LDS to add
// their sums in wave order. The x columns are read straight from memory: they are small and every
// work-group reads the same ones (L2-resident after the first).
//
// HBM-bound: per weight 2 (F16, BF16) or 4 (F32) bytes against 1 conversion and N fused
// multiply-adds.
#include "kernels.h"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdio>
#include <cstring>

namespace sgk {
namespace {

constexpr int kRows = 8;     // rows per work-group
constexpr int kStepK = 512;  // elements of K per wave step (8 per lane)

struct MvfArgs {
    MatArgs a;     // mats[0]; a.nb is the row stride in bytes
    int nmat;
    int64_t mt[4];  // matrix j owns work-groups mt[j] .. mt[j + 1]
    const uint8_t * wm[3];
    int64_t Mm[3];
    float * ym[3];
    int64_t ys1m[3];
    IdArgs id;     // MUL_MAT_ID (has_id): blockIdx.y is the pair t * n_used + i
    int has_id;
};

// 16 bytes of weights, non-temporal (read once per product, as in the quantized matvec)
typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16_nt(const uint8_t * p) {
    const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 8 consecutive weights of one row as f32 (p 16-byte aligned)
template <int WT> struct WLoad;
template <> struct WLoad<F32> {
    uint4 u, v;
    __device__ void load(const uint8_t * p) {
        u = ld16_nt(p);
        v = ld16_nt(p + 16);
    }
    __device__ void to_f32(float * o) const {
        o[0] = __uint_as_float(u.x), o[1] = __uint_as_float(u.y), o[2] = __uint_as_float(u.z), o[3] = __uint_as_float(u.w);
        o[4] = __uint_as_float(v.x), o[5] = __uint_as_float(v.y), o[6] = __uint_as_float(v.z), o[7] = __uint_as_float(v.w);
    }
};
template <> struct WLoad<F16> {
    uint4 q;
    __device__ void load(const uint8_t * p) { q = ld16_nt(p); }
    __device__ void to_f32(float * o) const {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = __half2float(__ushort_as_half((unsigned short) (w[i] & 0xFFFFu)));
            o[2 * i + 1] = __half2float(__ushort_as_half((unsigned short) (w[i] >> 16)));
        }
    }
};
template <> struct WLoad<BF16> {
    uint4 q;
    __device__ void load(const uint8_t * p) { q = ld16_nt(p); }
    __device__ void to_f32(float * o) const {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = __uint_as_float(w[i] << 16);
            o[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    }
};

// reduce-scatter of V = 2^P values over the wave's 64 lanes: afterwards lane l holds, in v[0], the
// sum over all lanes of value index_of(l)
template <int V>
__device__ inline void reduce_scatter(float (&v)[V], int lane) {
#pragma unroll
    for (int s = 0, n = V; n > 1; ++s, n >>= 1) {
        const int b = 32 >> s;
        const bool hi = (lane & b) != 0;
#pragma unroll
        for (int i = 0; i < n / 2; ++i) {
            const float send = hi ? v[i] : v[i + n / 2];
            const float keep = hi ? v[i + n / 2] : v[i];
            v[i] = keep + __shfl_xor(send, b);
        }
    }
#pragma unroll
    for (int b = 32 >> __builtin_ctz(V); b >= 1; b >>= 1) v[0] += __shfl_xor(v[0], b);
}

template <int V>
__device__ inline int index_of(int lane) {
    int idx = 0;
#pragma unroll
    for (int s = 0, n = V; n > 1; ++s, n >>= 1)
        if (lane & (32 >> s)) idx += n / 2;
    return idx;
}

// XV: x columns 16-byte aligned (vector loads), else scalar loads
template <int WT, int NC, bool XV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, NC >= 4 ? 2 : 4))) void k_mvf(MvfArgs A) {
    constexpr int V = kRows * NC;
    constexpr int U = WT == F32 || NC >= 4 ? 1 : 2; // steps whose loads are in flight together
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t tile = blockIdx.x, sl = blockIdx.y;
    const MatArgs & a = A.a;
    const int j = A.nmat == 1 ? 0 : (tile >= A.mt[1] ? (tile >= A.mt[2] ? 2 : 1) : 0);
    const int64_t M = A.nmat > 1 ? A.Mm[j] : a.M, m0 = (tile - A.mt[j]) * kRows;
    const int64_t i2 = sl % a.ne12, i3 = sl / a.ne12;
    const uint8_t * w = A.nmat > 1 ? A.wm[j] : a.w + (uint64_t) (i2 / a.r2) * a.w_s2 + (uint64_t) (i3 / a.r3) * a.w_s3;
    const float * x = a.x + i2 * a.x_s2 + i3 * a.x_s3;
    float * yb = A.nmat > 1 ? A.ym[j] : a.y + i2 * a.y_s2 + i3 * a.y_s3;
    if (A.has_id) {
        // the pair's expert (read on the device, clamped into range), x column and y column
        const int64_t t = sl / A.id.n_used, i = sl - t * A.id.n_used;
        int64_t e = A.id.ids[i * A.id.s0 + t * A.id.s1];
        e = e < 0 ? 0 : (e >= A.id.n_exp ? A.id.n_exp - 1 : e);
        w = (A.nmat > 1 ? A.wm[j] : a.w) + (uint64_t) e * a.w_s2;
        x = a.x + (A.id.x_shared ? 0 : i) * a.x_s1 + t * a.x_s2;
        yb = (A.nmat > 1 ? A.ym[j] : a.y) + i * a.y_s1 + t * a.y_s2;
    }
    const int64_t K = a.K, N = a.N;
    constexpr int esz = WT == F32 ? 4 : 2;
    const uint8_t * row[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) row[r] = w + (uint64_t) min<int64_t>(m0 + r, M - 1) * (uint64_t) a.nb;
    const float * xc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) xc[c] = x + min<int64_t>(c, N - 1) * a.x_s1;

    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;
    const int64_t steps = (K + kStepK - 1) / kStepK;
    for (int64_t s0 = wave; s0 < steps; s0 += 4 * U) {
        WLoad<WT> wl[U][kRows];
        float4 xl[U][NC][2];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t k = (s0 + 4 * u) * kStepK + 8 * lane;
            ok[u] = s0 + 4 * u < steps && k < K;
            const int64_t kc = min<int64_t>(k, K - 8); // (K is a multiple of 8; lanes past it are masked)
#pragma unroll
            for (int r = 0; r < kRows; ++r) wl[u][r].load(row[r] + kc * esz);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                if (XV) {
                    xl[u][c][0] = *reinterpret_cast<const float4 *>(xc[c] + kc);
                    xl[u][c][1] = *reinterpret_cast<const float4 *>(xc[c] + kc + 4);
                } else {
                    const float * q = xc[c] + kc;
                    xl[u][c][0] = make_float4(q[0], q[1], q[2], q[3]);
                    xl[u][c][1] = make_float4(q[4], q[5], q[6], q[7]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (!ok[u]) continue;
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                float wf[8];
                wl[u][r].to_f32(wf);
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const float xv[8] = {xl[u][c][0].x, xl[u][c][0].y, xl[u][c][0].z, xl[u][c][0].w,
                                         xl[u][c][1].x, xl[u][c][1].y, xl[u][c][1].z, xl[u][c][1].w};
                    float t = acc[r * NC + c];
#pragma unroll
                    for (int e = 0; e < 8; ++e) t = __builtin_fmaf(wf[e], xv[e], t);
                    acc[r * NC + c] = t;
                }
            }
        }
    }
    reduce_scatter<V>(acc, lane);
    __shared__ float red[4][V];
    red[wave][index_of<V>(lane)] = acc[0]; // (lanes holding the same index write the same sum)
    __syncthreads();
    const int t = threadIdx.x;
    if (t < V) {
        const int r = t / NC, c = t % NC;
        const float sum = ((red[0][t] + red[1][t]) + red[2][t]) + red[3][t];
        if (m0 + r < M && c < N) {
            const int64_t ys1 = A.nmat > 1 ? A.ys1m[j] : a.y_s1;
            yb[c * ys1 + m0 + r] = sum; // (MUL_MAT_ID: one column)
        }
    }
}

template <int WT, bool XV>
void * kernel_for(int nc) {
    return nc == 1 ? (void *) k_mvf<WT, 1, XV> : nc == 2 ? (void *) k_mvf<WT, 2, XV> : nc <= 4 ? (void *) k_mvf<WT, 4, XV> : (void *) k_mvf<WT, 8, XV>;
}

template <int WT>
void * kernel_for(int nc, bool xv) {
    return xv ? kernel_for<WT, true>(nc) : kernel_for<WT, false>(nc);
}

} // namespace

bool is_float_weight(int dtype) {
    return dtype == F32 || dtype == F16 || dtype == BF16;
}

hipError_t launch_matvec_float(const MatArgs * mats, int nmat, hipStream_t stream, const char ** kernel_name, uint64_t * grid_size,
                               const IdArgs * id) {
    if (nmat < 1 || nmat > 3) return hipErrorInvalidValue;
    if (id != nullptr && (mats[0].N != 1 || id->ids == nullptr || id->n_used < 1 || id->n_tok < 1 || id->n_exp < 1)) return hipErrorInvalidValue;
    if (mats[0].N > 8 && id == nullptr) {
        // more columns (F32 weights, or K not a whole number of GEMM stages): one launch per group
        // of 8 columns, each the exact product above
        for (int64_t c0 = 0; c0 < mats[0].N; c0 += 8) {
            MatArgs g[3];
            for (int j = 0; j < nmat; ++j) {
                g[j] = mats[j];
                g[j].N = std::min<int64_t>(8, mats[j].N - c0);
                g[j].x = mats[j].x + c0 * mats[j].x_s1;
                g[j].y = mats[j].y + c0 * mats[j].y_s1;
            }
            const hipError_t e = launch_matvec_float(g, nmat, stream, kernel_name, grid_size);
            if (e != hipSuccess) return e;
        }
        std::snprintf(last_form().form, sizeof(last_form().form), "float rows=8 column-groups=%d", (int) ((mats[0].N + 7) / 8));
        return hipSuccess;
    }
    const MatArgs & a = mats[0];
    if (!is_float_weight(a.dtype) || a.N < 1 || a.K < 8 || a.K % 8 != 0) return hipErrorInvalidValue;
    MvfArgs A;
    std::memset(&A, 0, sizeof(A));
    A.a = a;
    A.nmat = nmat;
    A.mt[0] = 0;
    for (int j = 0; j < 3; ++j) {
        const bool has = j < nmat;
        if (has && (mats[j].dtype != a.dtype || mats[j].K != a.K || mats[j].N != a.N || (nmat > 1 && id == nullptr && mats[j].ne12 * mats[j].ne13 != 1))) {
            return hipErrorInvalidValue;
        }
        A.wm[j] = has ? mats[j].w : nullptr;
        A.Mm[j] = has ? mats[j].M : 0;
        A.ym[j] = has ? mats[j].y : nullptr;
        A.ys1m[j] = has ? mats[j].y_s1 : 0;
        A.mt[j + 1] = A.mt[j] + (has ? (mats[j].M + kRows - 1) / kRows : 0);
    }
    if (id != nullptr) {
        A.id = *id;
        A.has_id = 1;
    }
    const int64_t slices = id != nullptr ? id->n_used * id->n_tok : a.ne12 * a.ne13;
    if (A.mt[nmat] > 0x7fffffff || slices > 65535) return hipErrorInvalidValue;
    const int nc = (int) a.N;
    const bool xv = (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && a.x_s1 % 4 == 0 && a.x_s2 % 4 == 0 && a.x_s3 % 4 == 0;
    void * fn = a.dtype == F32 ? kernel_for<F32>(nc, xv) : a.dtype == F16 ? kernel_for<F16>(nc, xv) : kernel_for<BF16>(nc, xv);
    const int ncp = nc == 1 ? 1 : nc == 2 ? 2 : nc <= 4 ? 4 : 8;
    const dim3 grid((unsigned) A.mt[nmat], (unsigned) slices);
    void * args[] = {&A};
    if (kernel_name) *kernel_name = a.dtype == F32 ? "matvec_f32" : a.dtype == F16 ? "matvec_f16" : "matvec_bf16";
    std::snprintf(last_form().form, sizeof(last_form().form), "float rows=%d nc=%d", kRows, ncp);
    last_form().grid = (uint64_t) grid.x * grid.y;
    if (grid_size) *grid_size = last_form().grid;
    return hipLaunchKernel(fn, grid, dim3(256), args, 0, stream);
}

} // namespace sgk
