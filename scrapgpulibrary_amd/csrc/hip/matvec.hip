// Decode matvec over R32 weights for 1 <= N <= 8 columns (gfx950, wave64).
//
// Work decomposition. A work-group (256 threads = 4 waves) owns one 32-row group of one slice and
// a contiguous range of "steps" along K (a step is one block: 32 elements of Q8_0, 256 of Q4_K /
// Q6_K; for Q4_0 a step is two blocks). Lane l of a wave serves row (l & 31) of the group; its
// half (l >> 5) selects which 16-byte units of the step it loads, so one wave-wide 128-bit load
// reads 2 x 512 contiguous bytes of the R32 area (fully coalesced). The 4 waves take the steps of
// the range round-robin.
//
// Arithmetic. A lane converts the bytes of a unit with one mask per 4 weights and one
// byte->float conversion per weight, then one FMA per weight and column against x from LDS
// (all 32 lanes of a half read the same LDS address: a broadcast). Block scales are factored out
// of the inner sum, and every constant offset of a format (Q4_0's -8, Q8_0's stored xor 0x80,
// Q6_K's -32, Q4_K's -dmin*m) is applied once per 16 weights through precomputed sums of 16
// consecutive x values (also in LDS):
//   Q4_0: d * (sum q x - 8 sum x)            Q8_0: d * (sum u x - 128 sum x)
//   Q4_K: d*sc * sum q x - dmin*m * sum x    Q6_K: d*sc * (sum q x - 32 sum x)
// The high nibble is used in place (value * 16) and the 1/16 folded into its scale.
//
// K split. When the row groups alone cannot fill the GPU, the K range is split over `ksplit`
// work-groups per row group. Each writes its partial sums to stream scratch; the last to arrive
// (an agent-scope atomic counter) adds the parts in part order -- deterministic -- writes y and
// re-arms the counter. One launch, no memset.
#include "kernels.h"

#include <hip/hip_fp16.h>

#include <algorithm>

namespace sgk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kLdsFloats = 16384; // 64 KiB of x (+ sums) per work-group at most

struct MvLaunch {
    MatArgs a;
    int64_t groups;
    int64_t steps;     // steps along K
    int64_t per_part;  // steps per work-group
    int ksplit;
    int elems_step;    // K elements per step
    float * partials;
    uint32_t * counters;
};

__device__ __forceinline__ float half_bits(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short) (h & 0xFFFFu)));
}

// sum over the 4 bytes of v of byte_i * x[i]
__device__ __forceinline__ float dot4(uint32_t v, float4 x, float acc) {
    acc = fmaf((float) (v & 0xFFu), x.x, acc);
    acc = fmaf((float) ((v >> 8) & 0xFFu), x.y, acc);
    acc = fmaf((float) ((v >> 16) & 0xFFu), x.z, acc);
    acc = fmaf((float) (v >> 24), x.w, acc);
    return acc;
}

// sum_i byte_i(q) * x[i] for the 16 bytes of q (already masked) and 16 floats of LDS
__device__ __forceinline__ float dot16(uint4 q, const float * xs) {
    const float4 * x4 = reinterpret_cast<const float4 *>(xs);
    float acc = 0.0f;
    acc = dot4(q.x, x4[0], acc);
    acc = dot4(q.y, x4[1], acc);
    acc = dot4(q.z, x4[2], acc);
    acc = dot4(q.w, x4[3], acc);
    return acc;
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

// ---- one step of one lane, per format ------------------------------------------------------
// xs: this work-group's x slab, column n at xs + n * xlen, element e at (e - e0);
// ss: sums of 16 consecutive x, column n at ss + n * nseg, segment (e - e0) / 16.

template <int NC>
__device__ __forceinline__ void step_q4_0(const MvLaunch & L, const uint8_t * w, int64_t g0, int rs, int row, int hf, int64_t s,
                                          int64_t e0, const float * xs, int xlen, const float * ss, int nseg, float * acc) {
    const int64_t b = 2 * s + hf;
    if (b >= L.a.nb) return;
    const int64_t nb = L.a.nb;
    const uint4 q = load16(w + (uint64_t) g0 * nb * 16 + ((uint64_t) b * rs + row) * 16);
    const uint32_t dh = *reinterpret_cast<const uint16_t *>(w + (uint64_t) L.a.M * nb * 16 + (uint64_t) g0 * nb * 2 + ((uint64_t) b * rs + row) * 2);
    const float d = half_bits(dh);
    const uint4 lo = mask4(q, 0x0F0F0F0Fu), hi = mask4(q, 0xF0F0F0F0u);
    const int off = (int) (32 * b - e0);
#pragma unroll
    for (int n = 0; n < NC; ++n) {
        const float * x = xs + n * xlen + off;
        const float * sm = ss + n * nseg + off / 16;
        const float t = (dot16(lo, x) - 8.0f * sm[0]) + (dot16(hi, x + 16) * 0.0625f - 8.0f * sm[1]);
        acc[n] = fmaf(d, t, acc[n]);
    }
}

template <int NC>
__device__ __forceinline__ void step_q8_0(const MvLaunch & L, const uint8_t * w, int64_t g0, int rs, int row, int hf, int64_t b,
                                          int64_t e0, const float * xs, int xlen, const float * ss, int nseg, float * acc) {
    const int64_t nb = L.a.nb;
    const uint4 u = load16(w + (uint64_t) g0 * nb * 32 + (((uint64_t) b * 2 + hf) * rs + row) * 16);
    const uint32_t dh = *reinterpret_cast<const uint16_t *>(w + (uint64_t) L.a.M * nb * 32 + (uint64_t) g0 * nb * 2 + ((uint64_t) b * rs + row) * 2);
    const float d = half_bits(dh);
    const int off = (int) (32 * b + 16 * hf - e0);
#pragma unroll
    for (int n = 0; n < NC; ++n) {
        const float t = dot16(u, xs + n * xlen + off) - 128.0f * ss[n * nseg + off / 16];
        acc[n] = fmaf(d, t, acc[n]);
    }
}

template <int NC>
__device__ __forceinline__ void step_q4_k(const MvLaunch & L, const uint8_t * w, int64_t g0, int rs, int row, int hf, int64_t b,
                                          int64_t e0, const float * xs, int xlen, const float * ss, int nseg, float * acc) {
    const int64_t nb = L.a.nb;
    const uint8_t * qb = w + (uint64_t) g0 * nb * 128 + ((uint64_t) b * 8 * rs + row) * 16;
    uint4 q[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) q[c] = load16(qb + (uint64_t) (2 * c + hf) * rs * 16);
    const uint4 hd = load16(w + (uint64_t) L.a.M * nb * 128 + (uint64_t) g0 * nb * 16 + ((uint64_t) b * rs + row) * 16);
    const float d = half_bits(hd.x), dmin = half_bits(hd.x >> 16);
    // 12 scale bytes s[0..11] = bytes 4..15 of the header
    const uint4 sv = make_uint4(hd.y, hd.z, hd.w, 0u);
    const int base = (int) (256 * b - e0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        uint32_t sc0, m0, sc1, m1;
        const int j0 = 2 * c, j1 = 2 * c + 1;
        if (c < 2) {
            sc0 = byte_of(sv, j0) & 63u;
            m0 = byte_of(sv, j0 + 4) & 63u;
            sc1 = byte_of(sv, j1) & 63u;
            m1 = byte_of(sv, j1 + 4) & 63u;
        } else {
            sc0 = (byte_of(sv, j0 + 4) & 0x0Fu) | ((byte_of(sv, j0 - 4) >> 6) << 4);
            m0 = (byte_of(sv, j0 + 4) >> 4) | ((byte_of(sv, j0) >> 6) << 4);
            sc1 = (byte_of(sv, j1 + 4) & 0x0Fu) | ((byte_of(sv, j1 - 4) >> 6) << 4);
            m1 = (byte_of(sv, j1 + 4) >> 4) | ((byte_of(sv, j1) >> 6) << 4);
        }
        const float dl = d * (float) sc0, ml = dmin * (float) m0;
        const float dhh = d * (float) sc1 * 0.0625f, mh = dmin * (float) m1;
        const uint4 lo = mask4(q[c], 0x0F0F0F0Fu), hi = mask4(q[c], 0xF0F0F0F0u);
        const int off = base + 64 * c + 16 * hf;
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            const float * x = xs + n * xlen + off;
            const float * sm = ss + n * nseg + off / 16;
            float a = acc[n];
            a = fmaf(dl, dot16(lo, x), a);
            a = fmaf(-ml, sm[0], a);
            a = fmaf(dhh, dot16(hi, x + 32), a);
            a = fmaf(-mh, sm[2], a);
            acc[n] = a;
        }
    }
}

template <int NC>
__device__ __forceinline__ void step_q6_k(const MvLaunch & L, const uint8_t * w, int64_t g0, int rs, int row, int hf, int64_t b,
                                          int64_t e0, const float * xs, int xlen, const float * ss, int nseg, float * acc) {
    const int64_t nb = L.a.nb, M = L.a.M;
    const uint8_t * qb = w + (uint64_t) g0 * nb * 192 + ((uint64_t) b * 12 * rs + row) * 16;
    const uint4 scv = load16(w + (uint64_t) M * nb * 192 + (uint64_t) g0 * nb * 16 + ((uint64_t) b * rs + row) * 16);
    const uint32_t dh = *reinterpret_cast<const uint16_t *>(w + (uint64_t) M * nb * 208 + (uint64_t) g0 * nb * 2 + ((uint64_t) b * rs + row) * 2);
    const float d = half_bits(dh);
    const int base = (int) (256 * b - e0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint4 qa = load16(qb + (uint64_t) (4 * h + hf) * rs * 16);     // ql[64h + 16hf + i]
        const uint4 qc = load16(qb + (uint64_t) (4 * h + 2 + hf) * rs * 16); // ql[64h + 32 + 16hf + i]
        const uint4 qh = load16(qb + (uint64_t) (8 + 2 * h + hf) * rs * 16); // qh[32h + 16hf + i]
        uint4 v[4];
        v[0] = make_uint4((qa.x & 0x0F0F0F0Fu) | ((qh.x << 4) & 0x30303030u), (qa.y & 0x0F0F0F0Fu) | ((qh.y << 4) & 0x30303030u),
                          (qa.z & 0x0F0F0F0Fu) | ((qh.z << 4) & 0x30303030u), (qa.w & 0x0F0F0F0Fu) | ((qh.w << 4) & 0x30303030u));
        v[1] = make_uint4((qc.x & 0x0F0F0F0Fu) | ((qh.x << 2) & 0x30303030u), (qc.y & 0x0F0F0F0Fu) | ((qh.y << 2) & 0x30303030u),
                          (qc.z & 0x0F0F0F0Fu) | ((qh.z << 2) & 0x30303030u), (qc.w & 0x0F0F0F0Fu) | ((qh.w << 2) & 0x30303030u));
        v[2] = make_uint4(((qa.x >> 4) & 0x0F0F0F0Fu) | (qh.x & 0x30303030u), ((qa.y >> 4) & 0x0F0F0F0Fu) | (qh.y & 0x30303030u),
                          ((qa.z >> 4) & 0x0F0F0F0Fu) | (qh.z & 0x30303030u), ((qa.w >> 4) & 0x0F0F0F0Fu) | (qh.w & 0x30303030u));
        v[3] = make_uint4(((qc.x >> 4) & 0x0F0F0F0Fu) | ((qh.x >> 2) & 0x30303030u), ((qc.y >> 4) & 0x0F0F0F0Fu) | ((qh.y >> 2) & 0x30303030u),
                          ((qc.z >> 4) & 0x0F0F0F0Fu) | ((qh.z >> 2) & 0x30303030u), ((qc.w >> 4) & 0x0F0F0F0Fu) | ((qh.w >> 2) & 0x30303030u));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            // scale byte 8h + 2r + hf, stored xor 0x80
            const int si = 8 * h + 2 * r + hf;
            const float sc = (float) (int8_t) (byte_of(scv, si) ^ 0x80u);
            const float ds = d * sc;
            const int off = base + 128 * h + 32 * r + 16 * hf;
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                const float t = dot16(v[r], xs + n * xlen + off) - 32.0f * ss[n * nseg + off / 16];
                acc[n] = fmaf(ds, t, acc[n]);
            }
        }
    }
}

template <int DT, int NC>
__global__ __launch_bounds__(kThreads) void k_matvec(MvLaunch L) {
    extern __shared__ float lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = lane & 31, hf = lane >> 5;
    const int64_t gi = blockIdx.x / L.ksplit;
    const int part = (int) (blockIdx.x % L.ksplit);
    const int64_t sl = blockIdx.y;
    const int64_t i2 = sl % L.a.ne12, i3 = sl / L.a.ne12;
    const uint8_t * w = L.a.w + (uint64_t) (i2 / L.a.r2) * L.a.w_s2 + (uint64_t) (i3 / L.a.r3) * L.a.w_s3;
    const float * x = L.a.x + i2 * L.a.x_s2 + i3 * L.a.x_s3;
    const int64_t g0 = gi * 32;
    const int rs = (int) min<int64_t>(32, L.a.M - g0);
    const int64_t s0 = part * L.per_part;
    const int64_t s1 = min<int64_t>(L.steps, s0 + L.per_part);
    const int64_t e0 = s0 * L.elems_step;
    const int64_t e1 = min<int64_t>(L.a.K, s1 * L.elems_step);
    const int xlen = (int) (e1 - e0);
    const int nseg = xlen / 16;
    float * xs = lds;
    float * ss = lds + NC * xlen;

    // stage x[e0, e1) of every column, then the sums of 16 consecutive values
    for (int i = tid; i < NC * xlen; i += kThreads) {
        const int n = i / xlen, e = i - n * xlen;
        xs[i] = x[n * L.a.x_s1 + e0 + e];
    }
    __syncthreads();
    for (int i = tid; i < NC * nseg; i += kThreads) {
        const int n = i / nseg, sg = i - n * nseg;
        const float4 * p = reinterpret_cast<const float4 *>(xs + n * xlen + 16 * sg);
        const float4 a = p[0], b = p[1], c = p[2], e = p[3];
        ss[i] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) + (((c.x + c.y) + (c.z + c.w)) + ((e.x + e.y) + (e.z + e.w)));
    }
    __syncthreads();

    float acc[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) acc[n] = 0.0f;
    if (row < rs) {
        for (int64_t s = s0 + wave; s < s1; s += kWaves) {
            if (DT == Q4_0) step_q4_0<NC>(L, w, g0, rs, row, hf, s, e0, xs, xlen, ss, nseg, acc);
            if (DT == Q8_0) step_q8_0<NC>(L, w, g0, rs, row, hf, s, e0, xs, xlen, ss, nseg, acc);
            if (DT == Q4_K) step_q4_k<NC>(L, w, g0, rs, row, hf, s, e0, xs, xlen, ss, nseg, acc);
            if (DT == Q6_K) step_q6_k<NC>(L, w, g0, rs, row, hf, s, e0, xs, xlen, ss, nseg, acc);
        }
    }
    // the two halves of a wave hold the same rows
#pragma unroll
    for (int n = 0; n < NC; ++n) acc[n] += __shfl_xor(acc[n], 32);

    __syncthreads(); // the x slab is reused as the reduction buffer
    float * red = lds;
    if (hf == 0) {
#pragma unroll
        for (int n = 0; n < NC; ++n) red[(wave * NC + n) * 32 + row] = acc[n];
    }
    __syncthreads();
    float v = 0.0f;
    const int n = tid >> 5, r = tid & 31;
    if (tid < NC * 32) {
        v = (red[(0 * NC + n) * 32 + r] + red[(1 * NC + n) * 32 + r]) + (red[(2 * NC + n) * 32 + r] + red[(3 * NC + n) * 32 + r]);
    }
    float * y = L.a.y + i2 * L.a.y_s2 + i3 * L.a.y_s3;
    if (L.ksplit == 1) {
        if (tid < NC * 32 && r < rs) y[n * L.a.y_s1 + g0 + r] = v;
        return;
    }
    const int64_t slot = sl * L.groups + gi;
    float * mine = L.partials + ((uint64_t) slot * L.ksplit + part) * (NC * 32);
    if (tid < NC * 32) mine[tid] = v;
    __threadfence();
    __syncthreads();
    __shared__ int last;
    if (tid == 0) {
        const uint32_t seen = __hip_atomic_fetch_add(L.counters + slot, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last = seen == (uint32_t) (L.ksplit - 1);
        if (last) __hip_atomic_store(L.counters + slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last || tid >= NC * 32 || r >= rs) return;
    const float * parts = L.partials + (uint64_t) slot * L.ksplit * (NC * 32);
    float t = 0.0f;
    for (int p = 0; p < L.ksplit; ++p) {
        t += __hip_atomic_load(parts + (uint64_t) p * (NC * 32) + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    y[n * L.a.y_s1 + g0 + r] = t;
}

template <int DT>
void * pick(int nc) {
    switch (nc) {
        case 1: return (void *) k_matvec<DT, 1>;
        case 2: return (void *) k_matvec<DT, 2>;
        case 3: return (void *) k_matvec<DT, 3>;
        case 4: return (void *) k_matvec<DT, 4>;
        case 5: return (void *) k_matvec<DT, 5>;
        case 6: return (void *) k_matvec<DT, 6>;
        case 7: return (void *) k_matvec<DT, 7>;
        default: return (void *) k_matvec<DT, 8>;
    }
}

const char * name_of(int dt) {
    switch (dt) {
        case Q4_0: return "matvec_q4_0";
        case Q8_0: return "matvec_q8_0";
        case Q4_K: return "matvec_q4_k";
        default: return "matvec_q6_k";
    }
}

} // namespace

hipError_t launch_matvec(const MatArgs & a, const Scratch & s, int cu_count, hipStream_t stream, const char ** kernel_name,
                         uint64_t * grid_size) {
    const int nc = (int) a.N;
    if (nc < 1 || nc > 8) return hipErrorInvalidValue;
    MvLaunch L;
    L.a = a;
    L.groups = (a.M + 31) / 32;
    L.elems_step = a.dtype == Q4_0 ? 64 : a.dtype == Q8_0 ? 32 : 256;
    L.steps = a.dtype == Q4_0 ? (a.nb + 1) / 2 : a.nb;
    const int64_t slices = a.ne12 * a.ne13;
    // enough work-groups for ~8 per CU, at least 4 steps (one per wave) per work-group, and an x
    // slab that fits the LDS budget
    const int64_t want = (int64_t) cu_count * 8;
    int64_t ksplit = 1;
    if (L.groups * slices < want) ksplit = (want + L.groups * slices - 1) / (L.groups * slices);
    ksplit = std::min<int64_t>(ksplit, std::max<int64_t>(1, L.steps / kWaves));
    const int64_t max_xlen = kLdsFloats / (nc + 1) / L.elems_step * L.elems_step;
    const int64_t min_split = (a.K + max_xlen - 1) / max_xlen;
    ksplit = std::max(ksplit, min_split);
    L.per_part = (L.steps + ksplit - 1) / ksplit;
    L.ksplit = (int) ((L.steps + L.per_part - 1) / L.per_part);
    if (L.ksplit > 1) {
        const uint64_t need_p = (uint64_t) L.groups * slices * L.ksplit * nc * 32;
        const uint64_t need_c = (uint64_t) L.groups * slices;
        if (need_p > s.partial_floats || need_c > s.counter_count) return hipErrorOutOfMemory;
    }
    L.partials = s.partials;
    L.counters = s.counters;
    const int64_t xlen = std::min<int64_t>(a.K, L.per_part * L.elems_step);
    const size_t lds = (size_t) std::max<int64_t>(nc * xlen + nc * (xlen / 16), kWaves * nc * 32) * sizeof(float);
    void * fn = nullptr;
    switch (a.dtype) {
        case Q4_0: fn = pick<Q4_0>(nc); break;
        case Q8_0: fn = pick<Q8_0>(nc); break;
        case Q4_K: fn = pick<Q4_K>(nc); break;
        case Q6_K: fn = pick<Q6_K>(nc); break;
        default: return hipErrorInvalidValue;
    }
    const dim3 grid((unsigned) (L.groups * L.ksplit), (unsigned) slices, 1);
    if (kernel_name) *kernel_name = name_of(a.dtype);
    if (grid_size) *grid_size = (uint64_t) grid.x * grid.y;
    void * args[] = {&L};
    return hipLaunchKernel(fn, grid, dim3(kThreads), args, lds, stream);
}

} // namespace sgk
