// Prefill matmul over R32 weights on the f16 MFMA units of gfx950 (fp32 accumulate), N > 8.
//
// Replaces, for the hip backend, the reference's tiled mat-mat kernels k_mm_* / k_mmx_*
// (src/backends/opencl11/kernels/mul_mm.cl:270-355, mul_mm_x.cl:437-539). Same product, new design:
//
//   pre-pass  x (fp32, any row stride) -> f16 rows [slice][N][K] in stream scratch, each token
//             row scaled by a power of two that puts its largest magnitude in [2^14, 2^15) (no
//             f16 overflow, no precision lost to subnormals); the factor is undone on the products.
//   GEMM      v_mfma_f32_32x32x16_f16 (the 32x32 tile sustains the chip's f16 rate; 16x16x32
//             issues at about half of it). A work-group is W waves (4, or 12 = one per CU); wave w
//             owns RG groups of 32 weight rows and BN tokens and walks K in stages of 128, the
//             stages unrolled by 4 so that every position-dependent choice is static.
//               * B operand (weights): lane (j, h) of a 32-row group holds row j, k-half h. Per
//                 stage it loads the R32 units of row j that hold its 64 codes, and dequantizes 8
//                 of them per k-step straight into f16 (see "weight codes" below). No weight goes
//                 through LDS and every weight is dequantized once per work-group. Q4_K takes one
//                 fma per f16 pair; its sub-block offsets enter through one extra MFMA per 4 stages.
//               * A operand (activations): the BN x 128 f16 x tile of the stage, double-buffered in
//                 LDS (XOR-swizzled 16-byte chunks); one ds_read_b128 per lane per MFMA, shared by
//                 the wave's RG row groups. The k order inside a step is whatever the weight lanes
//                 hold; the A reads follow it (chunk(h, t) below).
//             The next stage's weights and the x tile two stages ahead (BN = 64) are loaded into
//             registers while the current stage computes, every load outside branches; one
//             barrier per stage.
//   split-K   when the tiles alone leave CUs idle, K is split over work-groups that write partial
//             sums to scratch; a reduction kernel adds them in split order (deterministic).
#include "kernels.h"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <type_traits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

namespace sgk {
namespace {

constexpr int BK = 128;
constexpr int kChunks = BK / 8; // 16-byte chunks per LDS row of the x tile

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float half_bits(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short) (h & 0xFFFFu)));
}

__device__ __forceinline__ uint4 load16(const uint8_t * p) {
    return *reinterpret_cast<const uint4 *>(p);
}

__device__ __forceinline__ uint32_t load_u16(const uint8_t * p) {
    return *reinterpret_cast<const uint16_t *>(p);
}

__device__ __forceinline__ f16x2 h2(float v) {
    const _Float16 h = (_Float16) v;
    return f16x2{h, h};
}

__device__ __forceinline__ f16x2 as_h2(uint32_t v) {
    return __builtin_bit_cast(f16x2, v);
}

__device__ __forceinline__ uint32_t mad24(uint32_t a, uint32_t b, uint32_t c) {
    return __umul24(a, b) + c;
}

// ---- weight codes -> f16 B operands ----------------------------------------------------------
// A code c (0..255) in the low byte of a 16-bit half or'ed with 0x6400 reads as the f16 value
// 1024 + c exactly (f16 spacing is 1 on [1024, 2048)), so one v_and_or_b32 (or v_perm_b32) turns
// two codes into an f16 pair, and one packed add (or a packed fma for a code held 4 bits up:
// (1024 + 16c) / 16 - 64 = c) recovers the integers themselves. The scale is then one packed fma.
// Every B fragment holds the 8 elements e0..e7 of a run in the order e0 e2 e1 e3 e4 e6 e5 e7 (the
// pairs a dword of 4 byte codes gives), and the x rows in scratch carry the same order.
__device__ __forceinline__ uint32_t codes2(uint32_t v, uint32_t mask) {
    // one v_and_or_b32 (the compiler splits it when both constants are literals); the magic
    // lives in a VGPR, the mask in an SGPR: one constant-bus operand
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(0x64006400u));
    return r;
}

// bytes 0, 2 / 1, 3 of w as the f16 pairs 1024 + byte
__device__ __forceinline__ uint32_t bytes02(uint32_t w) {
    return __builtin_amdgcn_perm(0x64646464u, w, 0x04020400u);
}
__device__ __forceinline__ uint32_t bytes13(uint32_t w) {
    return __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u);
}

// f16 pair s * (h + bias) + o for an f16 pair h of integers (exact up to the fma's rounding)
__device__ __forceinline__ uint32_t affine(uint32_t h, f16x2 bias, f16x2 s, f16x2 o) {
    const f16x2 c = as_h2(h) + bias;
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, s, o));
}
__device__ __forceinline__ uint32_t affine16(uint32_t h, f16x2 bias, f16x2 s, f16x2 o) {
    const f16x2 c = __builtin_elementwise_fma(as_h2(h), f16x2{(_Float16) 0.0625f, (_Float16) 0.0625f}, bias);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, s, o));
}

// 4-bit codes of the dwords w0, w1 (low nibbles, or high nibbles when HI) -> 8 f16 s * (c + cb) + o
template <bool HI>
__device__ __forceinline__ f16x8 nib8(uint32_t w0, uint32_t w1, _Float16 cb, f16x2 s, f16x2 o) {
    const uint32_t mask = HI ? 0x00F000F0u : 0x000F000Fu;
    uint4 v;
    if constexpr (HI) {
        const f16x2 b = f16x2{(_Float16) (cb - (_Float16) 64.0f), (_Float16) (cb - (_Float16) 64.0f)};
        v.x = affine16(codes2(w0, mask), b, s, o);
        v.y = affine16(codes2(w0 >> 8, mask), b, s, o);
        v.z = affine16(codes2(w1, mask), b, s, o);
        v.w = affine16(codes2(w1 >> 8, mask), b, s, o);
    } else {
        const f16x2 b = f16x2{(_Float16) (cb - (_Float16) 1024.0f), (_Float16) (cb - (_Float16) 1024.0f)};
        v.x = affine(codes2(w0, mask), b, s, o);
        v.y = affine(codes2(w0 >> 8, mask), b, s, o);
        v.z = affine(codes2(w1, mask), b, s, o);
        v.w = affine(codes2(w1 >> 8, mask), b, s, o);
    }
    return __builtin_bit_cast(f16x8, v);
}

// byte codes of the dwords w0, w1 -> 8 f16 s * (c + cb)
__device__ __forceinline__ f16x8 byte8(uint32_t w0, uint32_t w1, _Float16 cb, f16x2 s) {
    const f16x2 b = f16x2{(_Float16) (cb - (_Float16) 1024.0f), (_Float16) (cb - (_Float16) 1024.0f)};
    const f16x2 z = f16x2{(_Float16) 0.0f, (_Float16) 0.0f};
    uint4 v;
    v.x = affine(bytes02(w0), b, s, z);
    v.y = affine(bytes13(w0), b, s, z);
    v.z = affine(bytes02(w1), b, s, z);
    v.w = affine(bytes13(w1), b, s, z);
    return __builtin_bit_cast(f16x8, v);
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

// ---- per format: one stage (128 elements of K) of one weight row for k-half h ----------------
// init() resolves the lane's row and k-half once into 32-bit byte offsets from the slice's weight
// base (one slice of weights is < 4 GiB, checked on the host) and the R32 unit stride
// U = 16 * rows-in-group; load(w, s) fetches the lane's bytes of stage s into a Raw (24-bit
// multiply-adds for the addresses); prep() turns a Raw's block scales into the stage's f16 factors;
// bop(raw, sc, t) is the lane's B fragment (8 f16) for k-step t = 0..7; chunk(h, t) is the 16-byte
// chunk (8 elements) of the stage's x row that the fragment pairs with.

template <int DT> struct PFmt;

// Q4_K: stage s = 64-element groups 2 (s % 2), 2 (s % 2) + 1 of block s / 2; k-half h takes group
// c = 2 (s % 2) + h, i.e. its two 16-byte units (bytes 0..31 of the group). k-step t: low (t < 4)
// or high nibbles of bytes 8 (t % 4) .. +7 = elements 64c + 8t + e of the block.
template <> struct PFmt<Q4_K> {
    struct Raw {
        uint4 q0, q1, hd;
    };
    // s: scale of the stage's two sub-blocks; o: their offsets (the exact form); n = -1024 s
    // (exact in f16) for the single-fma form; om: the offsets times 32 as an f16 pair, the lane's
    // two entries of the offset MFMA; big: a scale or offset too large for the single-fma form.
    // prep(.., g) returns the factors of the row scaled by the power of two g (see k_matmul).
    struct Sc {
        f16x2 s0, o0, s1, o1, n0, n1;
        uint32_t om;
        bool big;
    };
    uint32_t qo, ho, u;
    int h;
    __device__ void init(int64_t M, int64_t nb, const RowAddr & ra, int h_) {
        h = h_;
        u = ra.rs * 16;
        qo = (uint32_t) (ra.g0 * nb * 128 + ra.lr * 16) + 2 * h * u;
        ho = (uint32_t) (M * nb * 128 + ra.g0 * nb * 16 + ra.lr * 16);
    }
    // a block is 8 units; stage s starts at unit 4s
    __device__ Raw load(const uint8_t * w, int s) const {
        const uint32_t q = mad24((uint32_t) s * 4, u, qo);
        return Raw{load16(w + q), load16(w + (q + u)), load16(w + mad24((uint32_t) (s >> 1), u, ho))};
    }
    // stage s = the second half of prev's block: the header is prev's
    __device__ Raw load_half2(const uint8_t * w, int s, const Raw & prev) const {
        const uint32_t q = mad24((uint32_t) s * 4, u, qo);
        return Raw{load16(w + q), load16(w + (q + u)), prev.hd};
    }
    __device__ Sc prep(const Raw & r, int s, float g = 1.0f) const {
        const int c = 2 * (int) (s & 1) + h;
        const float d = g * half_bits(r.hd.x), dmin = g * half_bits(r.hd.x >> 16);
        float sc0, m0, sc1, m1;
        k4_scale_min(r.hd, 2 * c, sc0, m0);
        k4_scale_min(r.hd, 2 * c + 1, sc1, m1);
        const float fs0 = d * sc0, fs1 = d * sc1, fo0 = -32.0f * dmin * m0, fo1 = -32.0f * dmin * m1;
        Sc r0;
        r0.s0 = h2(fs0);
        r0.s1 = h2(fs1);
        r0.o0 = h2(-(dmin * m0));
        r0.o1 = h2(-(dmin * m1));
        const f16x2 k = f16x2{(_Float16) -1024.0f, (_Float16) -1024.0f};
        r0.n0 = r0.s0 * k;
        r0.n1 = r0.s1 * k;
        r0.om = __builtin_bit_cast(uint32_t, (f16x2{(_Float16) fo0, (_Float16) fo1}));
        // |d sc| <= 63 |d| < 32 and |32 dmin m| <= 2016 |dmin| < 32768 (a bound per block)
        r0.big = !(__builtin_fabsf(d) < 0.5f && __builtin_fabsf(dmin) < 16.0f);
        return r0;
    }
    // exact form: s (c + bias) + o per pair (low nibbles: s0, o0; high nibbles: s1, o1)
    __device__ static f16x8 bop(const Raw & r, const Sc & c, int t) {
        const uint4 & q = (t & 3) < 2 ? r.q0 : r.q1;
        const uint32_t w0 = (t & 1) ? q.z : q.x, w1 = (t & 1) ? q.w : q.y;
        return t < 4 ? nib8<false>(w0, w1, (_Float16) 0.0f, c.s0, c.o0) : nib8<true>(w0, w1, (_Float16) 0.0f, c.s1, c.o1);
    }
    // single-fma form: fma(1024 + c, s, -1024 s) = s c with one rounding (the addend is exact
    // while |s| < 64); a high nibble arrives as 1024 + 16 c and gives 16 s c, which pairs with x
    // stored divided by 16 at those positions. The offsets go through the offset MFMA instead.
    __device__ static f16x8 bop_fast(const Raw & r, const Sc & c, int t) {
        const uint4 & q = (t & 3) < 2 ? r.q0 : r.q1;
        const uint32_t w0 = (t & 1) ? q.z : q.x, w1 = (t & 1) ? q.w : q.y;
        const uint32_t mask = t < 4 ? 0x000F000Fu : 0x00F000F0u;
        const f16x2 sc = t < 4 ? c.s0 : c.s1, nb = t < 4 ? c.n0 : c.n1;
        uint4 v;
        v.x = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(as_h2(codes2(w0, mask)), sc, nb));
        v.y = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(as_h2(codes2(w0 >> 8, mask)), sc, nb));
        v.z = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(as_h2(codes2(w1, mask)), sc, nb));
        v.w = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(as_h2(codes2(w1 >> 8, mask)), sc, nb));
        return __builtin_bit_cast(f16x8, v);
    }
    __device__ static int chunk(int h, int t) {
        return 8 * h + t;
    }
};

// Q6_K: stage s = half n = s % 2 of block s / 2 (128 elements: runs rr = 0..3 of 32). k-half h
// takes elements l = 16h .. 16h + 15 of every run: units ql 4n + h (runs 0, 2), ql 4n + 2 + h
// (runs 1, 3), qh 8 + 2n + h. k-step t: run rr = t / 2, elements 32rr + 16h + 8 (t % 2) + e.
template <> struct PFmt<Q6_K> {
    struct Raw {
        uint4 qa, qc, qh, sc;
        uint32_t d;
    };
    struct Sc {
        f16x2 s[4];
    };
    uint32_t qo, so, dof, u;
    int h;
    __device__ void init(int64_t M, int64_t nb, const RowAddr & ra, int h_) {
        h = h_;
        u = ra.rs * 16;
        qo = (uint32_t) (ra.g0 * nb * 192 + ra.lr * 16) + h * u;
        so = (uint32_t) (M * nb * 192 + ra.g0 * nb * 16 + ra.lr * 16);
        dof = (uint32_t) (M * nb * 208 + ra.g0 * nb * 2 + ra.lr * 2);
    }
    // a block is 12 quant units (ql 0..7, qh 8..11), 1 scale unit and the d halves
    __device__ Raw load(const uint8_t * w, int s) const {
        const uint32_t b = (uint32_t) (s >> 1), n = (uint32_t) (s & 1);
        Raw r;
        const uint32_t qa = mad24(12 * b + 4 * n, u, qo);
        r.qa = load16(w + qa);                                 // ql[64n + l]
        r.qc = load16(w + qa + 2 * u);                         // ql[64n + 32 + l]
        r.qh = load16(w + mad24(12 * b + 8 + 2 * n, u, qo)); // qh[32n + l]
        r.sc = load16(w + mad24(b, u, so));
        r.d = load_u16(w + mad24(b, u >> 3, dof));
        return r;
    }
    // stage s = the second half of prev's block: the scales and d are prev's
    __device__ Raw load_half2(const uint8_t * w, int s, const Raw & prev) const {
        const uint32_t b = (uint32_t) (s >> 1), n = (uint32_t) (s & 1);
        Raw r;
        const uint32_t qa = mad24(12 * b + 4 * n, u, qo);
        r.qa = load16(w + qa);
        r.qc = load16(w + qa + 2 * u);
        r.qh = load16(w + mad24(12 * b + 8 + 2 * n, u, qo));
        r.sc = prev.sc;
        r.d = prev.d;
        return r;
    }
    // the signed 8-bit scale of run rr sits at byte 8n + h + 2rr (stored xor 0x80): word 2n (runs
    // 0, 1) or 2n + 1 (runs 2, 3), byte h or h + 2
    __device__ Sc prep(const Raw & r, int s) const {
        const uint32_t lo = (s & 1) ? r.sc.z : r.sc.x, hi = (s & 1) ? r.sc.w : r.sc.y;
        const int sh = 8 * h;
        const float d = half_bits(r.d);
        Sc c;
        c.s[0] = h2(d * ((float) ((lo >> sh) & 0xFFu) - 128.0f));
        c.s[1] = h2(d * ((float) ((lo >> (sh + 16)) & 0xFFu) - 128.0f));
        c.s[2] = h2(d * ((float) ((hi >> sh) & 0xFFu) - 128.0f));
        c.s[3] = h2(d * ((float) ((hi >> (sh + 16)) & 0xFFu) - 128.0f));
        return c;
    }
    // 6-bit codes of run rr: nibble rr / 2 of ql (qa for even rr, qc for odd), bits 2rr, 2rr + 1 of qh
    __device__ static f16x8 bop(const Raw & r, const Sc & c, int t) {
        const int rr = t >> 1;
        const uint4 & ql = (rr & 1) ? r.qc : r.qa;
        const int ls = 4 * (rr >> 1), hs = 2 * rr;
        const uint32_t l0 = (t & 1) ? ql.z : ql.x, l1 = (t & 1) ? ql.w : ql.y;
        const uint32_t h0 = (t & 1) ? r.qh.z : r.qh.x, h1 = (t & 1) ? r.qh.w : r.qh.y;
        const uint32_t v0 = ((l0 >> ls) & 0x0F0F0F0Fu) | (((h0 >> hs) << 4) & 0x30303030u);
        const uint32_t v1 = ((l1 >> ls) & 0x0F0F0F0Fu) | (((h1 >> hs) << 4) & 0x30303030u);
        return byte8(v0, v1, (_Float16) -32.0f, c.s[rr]);
    }
    __device__ static int chunk(int h, int t) {
        return 4 * (t >> 1) + 2 * h + (t & 1);
    }
};

// Q8_0: stage s = blocks 4s .. 4s + 3; k-half h takes blocks 4s + 2h + j, j = 0, 1 (2 units and a
// d each). k-step t: block j = t / 4, bytes 8 (t % 4) .. +7 = elements 32 (2h + j) + 8 (t % 4) + e
// of the stage. Blocks past the end of the row read the last block with scale 0.
template <> struct PFmt<Q8_0> {
    struct Raw {
        uint4 q[4];
        uint32_t d; // d of block j in bits 16j
    };
    struct Sc {
        f16x2 s[2];
    };
    uint32_t qo, dof, u, last;
    int h;
    __device__ void init(int64_t M, int64_t nb, const RowAddr & ra, int h_) {
        h = h_;
        u = ra.rs * 16;
        qo = (uint32_t) (ra.g0 * nb * 32 + ra.lr * 16);
        dof = (uint32_t) (M * nb * 32 + ra.g0 * nb * 2 + ra.lr * 2);
        last = (uint32_t) (nb - 1);
    }
    // block b: units 2b, 2b + 1 at 2b U; its d at b U / 8 in the d area
    __device__ Raw load(const uint8_t * w, int s) const {
        const uint32_t b0 = (uint32_t) s * 4 + 2 * h;
        Raw r;
        r.d = 0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t b = min(b0 + j, last);
            const uint32_t q = mad24(2 * b, u, qo);
            r.q[2 * j] = load16(w + q);
            r.q[2 * j + 1] = load16(w + q + u);
            if (b0 + j <= last) r.d |= load_u16(w + mad24(b, u >> 3, dof)) << (16 * j);
        }
        return r;
    }
    // one block per stage: nothing to share between stages
    __device__ Raw load_half2(const uint8_t * w, int s, const Raw &) const { return load(w, s); }
    __device__ Sc prep(const Raw & r, int) const {
        return Sc{{h2(half_bits(r.d)), h2(half_bits(r.d >> 16))}};
    }
    __device__ static f16x8 bop(const Raw & r, const Sc & c, int t) {
        const uint4 & q = r.q[2 * (t >> 2) + ((t & 3) >> 1)];
        const uint32_t w0 = (t & 1) ? q.z : q.x, w1 = (t & 1) ? q.w : q.y;
        return byte8(w0, w1, (_Float16) -128.0f, c.s[t >> 2]); // stored xor 0x80: value = (u - 128) d
    }
    __device__ static int chunk(int h, int t) {
        return 8 * h + t;
    }
};

// Q4_0: stage s = blocks 4s .. 4s + 3; k-half h takes blocks 4s + 2h + j, j = 0, 1 (1 unit and a d
// each). k-step t: block j = t / 4; low (t % 4 < 2) or high nibbles of bytes 8 (t % 2) .. +7 =
// elements 32 (2h + j) + 8 (t % 4) + e of the stage.
template <> struct PFmt<Q4_0> {
    struct Raw {
        uint4 q[2];
        uint32_t d;
    };
    struct Sc {
        f16x2 s[2];
    };
    uint32_t qo, dof, u, last;
    int h;
    __device__ void init(int64_t M, int64_t nb, const RowAddr & ra, int h_) {
        h = h_;
        u = ra.rs * 16;
        qo = (uint32_t) (ra.g0 * nb * 16 + ra.lr * 16);
        dof = (uint32_t) (M * nb * 16 + ra.g0 * nb * 2 + ra.lr * 2);
        last = (uint32_t) (nb - 1);
    }
    __device__ Raw load(const uint8_t * w, int s) const {
        const uint32_t b0 = (uint32_t) s * 4 + 2 * h;
        Raw r;
        r.d = 0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t b = min(b0 + j, last);
            r.q[j] = load16(w + mad24(b, u, qo));
            if (b0 + j <= last) r.d |= load_u16(w + mad24(b, u >> 3, dof)) << (16 * j);
        }
        return r;
    }
    // one block per stage: nothing to share between stages
    __device__ Raw load_half2(const uint8_t * w, int s, const Raw &) const { return load(w, s); }
    __device__ Sc prep(const Raw & r, int) const {
        return Sc{{h2(half_bits(r.d)), h2(half_bits(r.d >> 16))}};
    }
    __device__ static f16x8 bop(const Raw & r, const Sc & c, int t) {
        const uint4 & q = r.q[t >> 2];
        const uint32_t w0 = (t & 1) ? q.z : q.x, w1 = (t & 1) ? q.w : q.y;
        const f16x2 z = f16x2{(_Float16) 0.0f, (_Float16) 0.0f};
        return (t & 3) < 2 ? nib8<false>(w0, w1, (_Float16) -8.0f, c.s[t >> 2], z) : nib8<true>(w0, w1, (_Float16) -8.0f, c.s[t >> 2], z);
    }
    __device__ static int chunk(int h, int t) {
        return 8 * h + t;
    }
};

// F16 / BF16 rows in the natural layout (float weights, K a multiple of the 128-element stage):
// stage s = elements 128 s .. + 127 of the row; k-step t takes elements 16 t .. + 15, k-half h
// the 16-byte chunk 2 t + h of them: the two lanes of a row read 32 contiguous bytes per load, so a
// wave's load touches 32 cache lines instead of 64 (as 8 chunks per lane, contiguous). The pairs are reordered to the x tile's
// element order 0 2 1 3 of each group of 4. BF16 feeds the bf16 MFMA (x then in bf16, see
// k_x_to_f16), F16 the f16 one; neither needs scales.
template <int DT> struct PFmtFloat {
    struct Raw {
        uint4 q[8];
    };
    struct Sc {};
    uint32_t ro;
    int h;
    // (nb: the row stride in bytes for float weights)
    __device__ void init(int64_t, int64_t nb, const RowAddr & ra, int h_) {
        h = h_;
        ro = (uint32_t) ((ra.g0 + ra.lr) * nb) + 16 * (uint32_t) h_;
    }
    __device__ Raw load(const uint8_t * w, int s) const {
        const uint8_t * p = w + (ro + (uint32_t) s * 256);
        Raw r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r.q[i] = load16(p + 32 * i);
        return r;
    }
    __device__ Raw load_half2(const uint8_t * w, int s, const Raw &) const { return load(w, s); }
    __device__ Sc prep(const Raw &, int) const { return Sc{}; }
    __device__ static f16x8 bop(const Raw & r, const Sc &, int t) {
        const uint4 & q = r.q[t];
        const uint4 o = make_uint4((q.x & 0xFFFFu) | (q.y << 16), (q.x >> 16) | (q.y & 0xFFFF0000u), (q.z & 0xFFFFu) | (q.w << 16),
                                   (q.z >> 16) | (q.w & 0xFFFF0000u));
        return __builtin_bit_cast(f16x8, o);
    }
    __device__ static int chunk(int h, int t) {
        return 2 * t + h;
    }
};
template <> struct PFmt<F16> : PFmtFloat<F16> {};
template <> struct PFmt<BF16> : PFmtFloat<BF16> {};

// the GEMM's matrix instruction: f16 operands, or bf16 ones (BF16 weights) carried in f16x8
template <int DT>
__device__ __forceinline__ f32x16 mma32(const f16x8 & a, const f16x8 & b, const f32x16 & c) {
    if constexpr (DT == BF16) return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

struct MmArgs {
    MatArgs a;
    const uint16_t * xb; // f16 activations [slices][N][K], each row scaled (k_x_to_f16)
    const float * xs;    // [slices][N]: the factor that undoes a row's scaling
    float * part;        // split-K partial sums [split][slices][N][M] (split > 1)
    const uint16_t * xsum; // Q4_K: per token, the f16 sums / 32 of its 32-element sub-blocks (k_x_to_f16)
    int64_t xsum_row;    // halves per token row of xsum (16 per 512 elements of K)
    int64_t tiles_m, tiles_n;
    int64_t stages;      // stages of K (BK elements each)
    int split;           // work-groups along K per tile
    int sk_g;            // stream-K (k_gemm_w<.., SK>): the work-groups sharing the tiles' stages
    // grouped MUL_MAT_ID (GA kernels): pair p = t * n_used + slot; pairs[] grouped by expert,
    // expert e's pairs at e_off[e] .. e_off[e + 1] and token tiles at t_start[e] .. t_start[e + 1];
    // x row of a pair: t * x_cols + (x_cols > 1 ? slot : 0); y of a pair: a.y + slot * a.y_s1 + t * a.y_s2
    const int32_t * pairs;
    const int32_t * e_off;
    const int32_t * t_start;
    int32_t n_used, n_exp, x_cols;
    // nmat weights sharing x (prefill MUL_MAT_MULTI; one slice when nmat > 1): matrix j owns row
    // tiles mt[j] .. mt[j + 1] and columns mo[j] .. mo[j + 1] of the split-K partials (entries
    // from nmat on repeat the totals); nmat = 1 mirrors `a`. packed: the row tiles run over all
    // matrices' rows end to end instead (every matrix but the last a whole number of a wave's
    // 32 RG rows), each wave taking the matrix its rows are in
    int nmat, packed;
    int64_t mt[4], mo[4];
    const uint8_t * wm[3];
    int64_t Mm[3];
    float * ym[3];
    int64_t ys1m[3];
};

// padded x tile rows (the wide GEMM): 16-byte chunk c of token n at n * XR + 8 c (f16). The 16
// bytes of padding put consecutive tokens 4 banks apart, so the 16 lanes of one ds_read_b128
// cycle (16 tokens, one chunk) cover all 64 banks, and a lane's 8 k-steps are immediate offsets.
constexpr int XR = BK + 8;

// x tile in LDS: row n (token), 16-byte chunk c at (n * kChunks + (c ^ (n & 15))) * 8 f16
__device__ __forceinline__ int xsw(int n, int c) {
    return (n * kChunks + (c ^ (n & 15))) * 8;
}

// the x tile of one stage: BN tokens x 16 chunks over the 64 W threads of the work-group; thread p
// loads chunk p % 16 of tokens tb + 4 W i, tb = (p / 16) % BN (a thread whose token i lies past
// the tile repeats its token tb: same data to the same LDS slot). Every load is unconditional, so that the
// compiler's wait counting stays exact (a load under a branch makes it wait for all loads in
// flight): tokens past N read token N - 1 (their products land in outputs that are never stored),
// and chunks past K read the row's last chunk and are zeroed when stored to LDS (the weights there
// are zero as well, but x could hold an infinity). GA: the tokens are gathered rows (init_rows).
template <int BN, int W, bool GA = false>
struct XTile {
    static constexpr int NP = (BN * kChunks + 64 * W - 1) / (64 * W);
    uint32_t offs[GA ? NP : 1]; // GA: byte offset of each load's (gathered row, chunk)
    static constexpr int TS = 4 * W; // tokens between a thread's loads
    uint32_t off;     // byte offset of (token p / 16, chunk p % 16) in the slice's x rows
    uint32_t last;    // the same for token N - 1 (tokens past N read it)
    uint32_t step;    // TS tokens
    uint32_t kc;      // element offset of the chunk inside a stage
    int kmax;         // K - 8 - kc: the stage offset at which the chunk is the row's last one
    int dst;
    int k0;           // the last load's stage start (wave-uniform)
    bool tail;        // ... which reaches past K
    uint4 v[NP];
    int p;            // the thread's index among the 64 W threads that load the tile
    int tb;           // its first token, (p / 16) % BN (more threads than chunks: repeats)
    __device__ void init(int64_t N, int64_t K, int64_t n0, int p_) {
        p = p_;
        tb = (p >> 4) % BN;
        kc = 8 * (p & 15);
        dst = xsw(tb, p & 15); // token + TS i keeps the swizzle when TS is a multiple of 16
        off = 2 * ((uint32_t) ((n0 + tb) * K) + kc);
        last = 2 * ((uint32_t) ((N - 1) * K) + kc);
        step = (uint32_t) (2 * TS * K);
        kmax = (int) K - 8 - (int) kc;
        k0 = 0;
        tail = false;
    }
    // GA: the tile's tokens are the x rows rows[0 .. BN) (gathered pairs, repeated past the count)
    __device__ void init_rows(int64_t K, const int32_t * rows, int p_) {
        p = p_;
        tb = (p >> 4) % BN;
        kc = 8 * (p & 15);
        dst = xsw(tb, p & 15);
        off = last = step = 0;
        kmax = (int) K - 8 - (int) kc;
        k0 = 0;
        tail = false;
#pragma unroll
        for (int i = 0; i < (GA ? NP : 1); ++i) {
            const int n = tb + TS * i;
            offs[i] = 2 * ((uint32_t) rows[n < BN ? n : tb] * (uint32_t) K + kc);
        }
    }
    // the stage starting at element k0
    // (32-bit byte offsets from the slice's base: one scalar base, no 64-bit address math)
    __device__ void load(const uint16_t * xb, int k0_, int K) {
        k0 = k0_;
        tail = k0 + BK > K;
        const uint32_t k = 2 * (uint32_t) min(k0, kmax); // chunks past K: the row's last chunk
        const uint8_t * base = reinterpret_cast<const uint8_t *>(xb);
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            if constexpr (GA) {
                v[i] = *reinterpret_cast<const uint4 *>(base + (offs[i] + k));
            } else {
                const uint32_t o = tb + TS * i < BN ? off + i * step : off;
                v[i] = *reinterpret_cast<const uint4 *>(base + (min(o, last) + k));
            }
        }
    }
    __device__ void store(uint16_t * X) {
        if (tail) { // the last stage of a K that is not a multiple of the stage
            const bool zero = k0 > kmax + 7; // k0 + kc >= K
#pragma unroll
            for (int i = 0; i < NP; ++i) v[i] = zero ? make_uint4(0, 0, 0, 0) : v[i];
        }
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int n = tb + TS * i;
            // (TS = 24 with 6 loading waves: the token's own swizzle)
            const int at = n < BN ? (TS % 16 == 0 ? dst + i * TS * BK : xsw(n, p & 15)) : dst;
            *reinterpret_cast<uint4 *>(X + at) = v[i];
        }
    }
};

// the B fragment of k-step t in the single-fma form (FAST: Q4_K) or the exact form (the others)
template <bool FAST, class F>
__device__ __forceinline__ f16x8 bop_of(const typename F::Raw & r, const typename F::Sc & c, int t) {
    if constexpr (FAST) return F::bop_fast(r, c, t);
    else return F::bop(r, c, t);
}

// work-groups of W waves per CU that the register file (and, at BN = 128, the LDS) holds
constexpr int occupancy_of(int dt, int bn, int rg, int w = 4) {
    // (float weights: 32 registers per stage of a row's raw data, held for two stages)
    return dt == F16 || dt == BF16 ? (w == 12 || bn > 64 || rg > 1 ? 1 : 2)
         : w == 12 ? 1 : bn == 32 ? 3 : bn == 64 && rg == 1 ? (dt == Q6_K ? 2 : 3) : bn == 128 && rg == 2 ? 1 : 2;
}

// W = 4: a work-group per SIMD quad, several per CU. W = 12: the CU's whole complement of 3 waves
// per SIMD in one work-group: its waves keep in step at the stage barrier, where separate
// work-groups on one CU drift apart (the oldest waves win the issue arbitration, so the last
// work-group finishes alone with one wave per SIMD). KG = 1: 12 row waves, a tile of 384 rows,
// each x tile serving 3x the rows; KG = 3: 4 row waves x 3 groups that take a third of K each
// (their own x tiles), added in LDS at the end (split-K without a second pass over memory).
// GA: grouped MUL_MAT_ID (KG = 1, no split): blockIdx.x = token tile * tiles_m + row tile;
// a token tile belongs to one expert, whose weights the work-group reads, and gathers its pairs'
// x rows / scatters their outputs through a table in LDS after the x buffers.
template <int DT, int BN, int RG, int W, int KG, bool GA = false>
__global__ __launch_bounds__(64 * W, occupancy_of(DT, BN, RG, W)) void k_matmul(MmArgs L) {
    constexpr int NF = BN / 32; // token fragments per wave
    constexpr int RW = W / KG;  // row waves
    constexpr int BMT = 32 * RG * RW;
    using F = PFmt<DT>;
    using Raw = typename F::Raw;
    struct RawSet {
        Raw r[RG];
    };
    extern __shared__ __attribute__((aligned(16))) uint16_t lds_mm[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = (tid >> 6) % RW, kg = (tid >> 6) / RW; // row wave, K group
    const int j = lane & 31, h = lane >> 5;
    const int64_t tile = blockIdx.x / L.split;
    const int split = (int) (blockIdx.x % L.split);
    const int64_t tm = tile % L.tiles_m, tn = tile / L.tiles_m;
    const int64_t sl = blockIdx.y;
    const int64_t i2 = sl % L.a.ne12, i3 = sl / L.a.ne12;
    // the wave's matrix (several when weights share x)
    const int64_t grow = tm * BMT + 32 * RG * wave; // packed: the wave's first row over all matrices
    const int mj = L.nmat == 1 ? 0
                 : L.packed    ? min(L.nmat - 1, grow >= L.mo[1] ? (grow >= L.mo[2] ? 2 : 1) : 0)
                               : (tm >= L.mt[1] ? (tm >= L.mt[2] ? 2 : 1) : 0);
    const uint8_t * w = L.nmat > 1 ? L.wm[mj] : L.a.w + (uint64_t) (i2 / L.a.r2) * L.a.w_s2 + (uint64_t) (i3 / L.a.r3) * L.a.w_s3;
    const int64_t K = L.a.K, nb = L.a.nb;
    const int64_t M = L.nmat > 1 ? L.Mm[mj] : L.a.M;
    int64_t N = L.a.N;
    int64_t n0 = tn * BN;
    const int64_t m0 = L.packed ? grow - L.mo[mj] : (tm - L.mt[mj]) * BMT + 32 * RG * wave;
    int32_t * ga_rows = reinterpret_cast<int32_t *>(lds_mm + KG * 2 * BN * BK); // GA: x row of tile token n
    int64_t * ga_y = reinterpret_cast<int64_t *>(ga_rows + BN);               // GA: its y element offset
    int32_t ga_cnt = BN;                                                      // GA: the tile's pairs
    bool half_tile = false;                                                   // GA: ga_cnt <= 32 (wave-uniform)
    if constexpr (GA) {
        // the expert owning token tile tn: the last e with t_start[e] <= tn (an empty expert
        // shares its start with the next one)
        if (tn >= L.t_start[L.n_exp]) return; // past this call's tiles (the whole work-group)
        int lo = 0, hi = L.n_exp - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (L.t_start[mid] <= tn) lo = mid;
            else hi = mid - 1;
        }
        const int32_t pb = L.e_off[lo] + (int32_t) (tn - L.t_start[lo]) * BN;
        ga_cnt = min(BN, L.e_off[lo + 1] - pb);
        half_tile = ga_cnt <= 32;
        w = L.a.w + (uint64_t) lo * L.a.w_s2;
        if (tid < BN) {
            const int32_t pr = L.pairs[pb + min(tid, ga_cnt - 1)]; // tokens past the count repeat the last pair
            const int32_t t = pr / L.n_used, slot = pr - t * L.n_used;
            ga_rows[tid] = t * L.x_cols + (L.x_cols > 1 ? slot : 0);
            ga_y[tid] = (int64_t) slot * L.a.y_s1 + (int64_t) t * L.a.y_s2;
        }
        __syncthreads();
        N = BN;
        n0 = 0;
    }
    // splits cover whole groups of 4 stages (the host keeps split <= groups), so a stage's
    // position in its group is (s - s0) % 4
    // (KG > 1, split 1: every K group walks gsz = 4 ceil(groups / KG) stages, so that all waves
    // meet the same barriers; stages past a group's share of K (s >= s1) are inactive: their loads
    // repeat a valid stage, their k-steps and offsets are skipped)
    const int64_t groups = (L.stages + 3) / 4;
    // (stage indices in 32 bits: K < 2^31 elements, and scalar 32-bit compares)
    const int gsz = (int) (4 * ((groups + KG - 1) / KG));
    const int s0 = (int) (KG > 1 ? kg * gsz : 4 * (groups * split / L.split));
    const int s1 = (int) (KG > 1 ? min<int64_t>(s0 + gsz, L.stages) : min(4 * (groups * (split + 1) / L.split), L.stages));
    const int send = KG > 1 ? s0 + gsz : s1;                      // the loop's end (KG > 1: the same count for all)
    const int lim = s1 > s0 ? s1 - 1 : (int) L.stages - 1;       // the last stage a load may read

    F f[RG];
#pragma unroll
    for (int i = 0; i < RG; ++i) f[i].init(M, nb, RowAddr(M, m0 + 32 * i + j), h);
    const uint16_t * xb = L.xb + (uint64_t) sl * N * K;
    XTile<BN, RW, GA> xt;
    if constexpr (GA) xt.init_rows(K, ga_rows, tid - kg * 64 * RW);
    else xt.init(N, K, n0, tid - kg * 64 * RW);
    uint16_t * const lds_x = lds_mm + kg * (2 * BN * BK); // the K group's two x buffers
    // LDS element offsets of the lane's A fragments: k-step t, token fragment q at aoff[t] + 32 q rows
    int aoff[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) aoff[t] = xsw(j, F::chunk(h, t));

    // Q4_K: the sub-block offsets o (the "min" term) are not folded into the B pairs but added by
    // one extra MFMA per 4 stages (2 blocks = 16 sub-blocks): A = the tokens' sub-block sums of x,
    // B = 32 o of the rows' sub-blocks. Lane (j, h) contributes the offsets of the two sub-blocks
    // it dequantizes each stage (dword s % 4 of bm); the xsum rows are ordered to match.
    constexpr bool kOff = DT == Q4_K;
    uint32_t bm[RG][4];
    f16x8 asum[NF];
    uint32_t soff[NF];
#pragma unroll
    for (int i = 0; i < RG; ++i)
#pragma unroll
        for (int d = 0; d < 4; ++d) bm[i][d] = 0u;
#pragma unroll
    for (int q = 0; q < NF; ++q) {
        const int64_t row = GA ? ga_rows[32 * q + j] : (int64_t) sl * N + min<int64_t>(n0 + 32 * q + j, N - 1);
        soff[q] = (uint32_t) (row * L.xsum_row) + 8 * h;
    }

    f32x16 acc[RG][NF];
#pragma unroll
    for (int i = 0; i < RG; ++i)
#pragma unroll
        for (int q = 0; q < NF; ++q)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][q][v] = 0.0f;

    // one stage: MFMAs over the x tile in LDS with the weights cw (row groups of the wave);
    // meanwhile the weights of stage s + 1 are loaded into nw and the x tile of stage s + XD into
    // xl, while xn (the x tile of stage s + 1) goes to the other LDS buffer at the end. XD = 2
    // (two register sets, xn loaded a stage earlier) where the registers allow it (BN = 64 with
    // one K group), else 1 (xl and xn are one set)
    constexpr int XD = BN == 64 && KG == 1 ? 2 : 1;
    // D = s % 4, a compile-time constant: the LDS buffer, the parity the formats' factors depend
    // on and the offset-MFMA slot are static
    auto stage = [&](auto dtag, int s, const RawSet & cw, RawSet & nw, XTile<BN, RW, GA> & xn, XTile<BN, RW, GA> & xl) __attribute__((always_inline)) {
        constexpr int D = decltype(dtag)::value;
        // past the split's last stage the loads repeat it (unused): no load sits under a branch.
        // The x sums of the group come first (waiting for them waits for nothing newer).
        if constexpr (kOff && D == 0) {
#pragma unroll
            for (int q = 0; q < NF; ++q)
                asum[q] = *reinterpret_cast<const f16x8 *>(reinterpret_cast<const uint8_t *>(L.xsum) + 2 * (soff[q] + (uint32_t) (min(s, lim) >> 2) * 16));
        }
        const int sn = min(s + 1, lim), sx = min(s + XD, lim);
#pragma unroll
        for (int i = 0; i < RG; ++i) {
            // K-quants: a stage is half a block; the odd half reuses the even half's block fields
            // (sn = s + 1 in the same block, or s itself at the end)
            if constexpr ((DT == Q4_K || DT == Q6_K) && (D & 1) == 0) nw.r[i] = f[i].load_half2(w, sn, cw.r[i]);
            else nw.r[i] = f[i].load(w, sn);
        }
        xl.load(xb, sx * BK, (int) K);
        const uint16_t * X = lds_x + (D & 1) * (BN * BK);
        const int sp = (s & ~3) | D; // = s, with its low bits visible to the compiler
        // an inactive stage (KG > 1, past the group's share of K) skips everything but its loads,
        // its x store and the barrier (a wave-uniform branch without global loads)
        if (KG == 1 || s < s1) {
        typename F::Sc sc[RG];
#pragma unroll
        for (int i = 0; i < RG; ++i) sc[i] = f[i].prep(cw.r[i], sp);
        // Q4_K, a row whose stage has a scale or offset too large for the single-fma form (rare:
        // weights in the hundreds): the row's factors are scaled by g = 2^-11 and its
        // accumulators by g for the stage (by 1 / g after it), and the stage's offsets are added
        // at once at that scale. Both lanes of a row (j, j + 32) agree on g; the branches are
        // wave-uniform and hold no loads.
        bool rare = false;
        float g = 1.0f;
        if constexpr (kOff) {
            bool big = false;
#pragma unroll
            for (int i = 0; i < RG; ++i) big = big || sc[i].big;
            rare = __builtin_amdgcn_ballot_w64(big) != 0;
            if (rare) {
                // the row's flag: either lane of it (the shuffle runs in every lane)
                const int partner = __shfl_xor((int) big, 32);
                g = big || partner != 0 ? 0.00048828125f : 1.0f;
#pragma unroll
                for (int i = 0; i < RG; ++i) {
                    sc[i] = f[i].prep(cw.r[i], sp, g);
                    // the group's pending offsets first, at the unscaled level
                    const f16x8 bo = __builtin_bit_cast(f16x8, make_uint4(bm[i][0], bm[i][1], bm[i][2], bm[i][3]));
#pragma unroll
                    for (int q = 0; q < NF; ++q) {
                        acc[i][q] = __builtin_amdgcn_mfma_f32_32x32x16_f16(asum[q], bo, acc[i][q], 0, 0, 0);
                        acc[i][q] *= g;
                    }
#pragma unroll
                    for (int dd = 0; dd < 4; ++dd) bm[i][dd] = 0u;
                }
            }
        }
        // software pipeline over the 8 k-steps: the A reads and B dequantization of step t + 1
        // are issued while the MFMAs of step t run
        f16x8 a[2][NF], b[2][RG];
#pragma unroll
        for (int q = 0; q < NF; ++q) a[0][q] = *reinterpret_cast<const f16x8 *>(X + aoff[0] + q * 32 * BK);
#pragma unroll
        for (int i = 0; i < RG; ++i) b[0][i] = bop_of<kOff, F>(cw.r[i], sc[i], 0);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int c = t & 1, n = c ^ 1;
            if (t < 7) {
#pragma unroll
                for (int q = 0; q < NF; ++q) a[n][q] = *reinterpret_cast<const f16x8 *>(X + aoff[t + 1] + q * 32 * BK);
            }
            __builtin_amdgcn_sched_barrier(0); // keep the reads ahead of this step's MFMAs
#pragma unroll
            for (int q = 0; q < NF; ++q) {
                // GA: a tile of at most 32 pairs leaves the second token fragment to padding
                if (GA && q > 0 && half_tile) continue;
#pragma unroll
                for (int i = 0; i < RG; ++i) acc[i][q] = mma32<DT>(a[c][q], b[c][i], acc[i][q]);
            }
            if (t < 7) {
#pragma unroll
                for (int i = 0; i < RG; ++i) b[n][i] = bop_of<kOff, F>(cw.r[i], sc[i], t + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (kOff) {
            // this stage's offsets (dword s % 4 of the offset operand); the offset MFMA runs when
            // the group of 4 stages or the split ends, or at once in a rare stage
#pragma unroll
            for (int i = 0; i < RG; ++i) bm[i][D] = sc[i].om;
            if (rare || D == 3 || s + 1 == s1) {
#pragma unroll
                for (int i = 0; i < RG; ++i) {
                    const f16x8 bo = __builtin_bit_cast(f16x8, make_uint4(bm[i][0], bm[i][1], bm[i][2], bm[i][3]));
#pragma unroll
                    for (int q = 0; q < NF; ++q) acc[i][q] = __builtin_amdgcn_mfma_f32_32x32x16_f16(asum[q], bo, acc[i][q], 0, 0, 0);
#pragma unroll
                    for (int dd = 0; dd < 4; ++dd) bm[i][dd] = 0u;
                }
            }
            if (rare) {
                const float ig = 1.0f / g;
#pragma unroll
                for (int i = 0; i < RG; ++i)
#pragma unroll
                    for (int q = 0; q < NF; ++q) acc[i][q] *= ig;
            }
        }
        } // active stage
        if (s + 1 < s1) xn.store(lds_x + ((D + 1) & 1) * (BN * BK));
        __syncthreads();
    };
    RawSet ra{}, rb{};
    XTile<BN, RW, GA> xt2 = xt;
    // every split has at least one stage (the host keeps split <= stages)
#pragma unroll
    for (int i = 0; i < RG; ++i) ra.r[i] = f[i].load(w, min(s0, lim));
    xt.load(xb, min(s0, lim) * BK, (int) K);
    if constexpr (XD == 2) xt2.load(xb, min(s0 + 1, lim) * BK, (int) K);
    xt.store(lds_x);
    __syncthreads();
    // groups of 4 stages, then the split's last 1..3 outside the loop (a stage under a branch
    // inside the loop would end every iteration with a wait for all loads in flight)
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    XTile<BN, RW, GA> & xa = XD == 2 ? xt2 : xt; // x set of stages D = 0, 2 (the next tile's)
    XTile<BN, RW, GA> & xc = xt;                 // of stages D = 1, 3
    int s = s0;
    for (; s + 3 < send; s += 4) {
        stage(I0{}, s, ra, rb, xa, xc);
        stage(I1{}, s + 1, rb, ra, xc, xa);
        stage(I2{}, s + 2, ra, rb, xa, xc);
        stage(I3{}, s + 3, rb, ra, xc, xa);
    }
    if (s < send) { // (KG > 1: send - s0 is a multiple of 4, no tail)
        stage(I0{}, s, ra, rb, xa, xc);
        if (s + 1 < s1) {
            stage(I1{}, s + 1, rb, ra, xc, xa);
            if (s + 2 < s1) stage(I2{}, s + 2, ra, rb, xa, xc);
        }
    }
    if constexpr (KG > 1) {
        // the K groups' sums, added in group order through LDS (the x buffers are free now):
        // red[(group - 1) * RW + wave][element][lane]
        constexpr int PER = RG * NF * 16;
        float * red = reinterpret_cast<float *>(lds_mm);
        __syncthreads();
        if (kg > 0) {
            float * r = red + ((size_t) ((kg - 1) * RW + wave) * PER) * 64 + lane;
#pragma unroll
            for (int i = 0; i < RG; ++i)
#pragma unroll
                for (int q = 0; q < NF; ++q)
#pragma unroll
                    for (int v = 0; v < 16; ++v) r[((i * NF + q) * 16 + v) * 64] = acc[i][q][v];
        }
        __syncthreads();
        if (kg > 0) return;
#pragma unroll
        for (int g = 1; g < KG; ++g) {
            const float * r = red + ((size_t) ((g - 1) * RW + wave) * PER) * 64 + lane;
#pragma unroll
            for (int i = 0; i < RG; ++i)
#pragma unroll
                for (int q = 0; q < NF; ++q)
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[i][q][v] += r[((i * NF + q) * 16 + v) * 64];
        }
    }
    // acc[i][q][v], lane (j, h): token n0 + 32q + 8 (v / 4) + 4h + v % 4, weight row m0 + 32i + j
    const int64_t slices = L.a.ne12 * L.a.ne13;
    float * y;
    int64_t ys1;
    if (L.split == 1) {
        y = L.nmat > 1 ? L.ym[mj] : L.a.y + i2 * L.a.y_s2 + i3 * L.a.y_s3;
        ys1 = L.nmat > 1 ? L.ys1m[mj] : L.a.y_s1;
    } else {
        const int64_t mt_all = L.mo[L.nmat]; // the partials' row length: all matrices' rows
        y = L.part + ((uint64_t) split * slices + (uint64_t) sl) * N * mt_all + L.mo[mj];
        ys1 = mt_all;
    }
    const float * xs = L.xs + (uint64_t) sl * N;
    if constexpr (GA) {
        // scatter: token n of the tile is pair ga_y[n] (the pairs past ga_cnt are not stored)
#pragma unroll
        for (int q = 0; q < NF; ++q) {
            float u[16];
#pragma unroll
            for (int v = 0; v < 16; ++v) u[v] = L.xs[ga_rows[32 * q + 8 * (v >> 2) + 4 * h + (v & 3)]];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int n = 32 * q + 8 * (v >> 2) + 4 * h + (v & 3);
                if (n >= ga_cnt) continue;
                float * yn = L.a.y + ga_y[n];
#pragma unroll
                for (int i = 0; i < RG; ++i) {
                    const int64_t m = m0 + 32 * i + j;
                    if (m < M) yn[m] = acc[i][q][v] * u[v];
                }
            }
        }
        return;
    }
#pragma unroll
    for (int q = 0; q < NF; ++q) {
        float u[16]; // the fragment's row factors, loaded together (tokens past N read N - 1)
#pragma unroll
        for (int v = 0; v < 16; ++v) u[v] = xs[min<int64_t>(n0 + 32 * q + 8 * (v >> 2) + 4 * h + (v & 3), N - 1)];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t n = n0 + 32 * q + 8 * (v >> 2) + 4 * h + (v & 3);
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < RG; ++i) {
                const int64_t m = m0 + 32 * i + j;
                if (m < M) y[n * ys1 + m] = acc[i][q][v] * u[v];
            }
        }
    }
}

// The wide GEMM's x tile, straight from the f16 rows into LDS (global_load_lds_dwordx4: lane i of
// one instruction writes 16 bytes at the instruction's LDS base + 16 i, no registers on the way).
// A token row is 17 slots of 16 bytes (16 chunks + the pad, which receives a second copy of chunk
// 15), so the 128-token tile is 2176 slots = exactly 34 wave instructions; LW loading waves take
// instructions w, w + LW, ...; a wave's index past the 34th repeats the 34th (the same bytes to the
// same slots). Tokens past N read token N - 1 (their products are never stored); K is a multiple
// of the stage, so no chunk lies past the row.
template <int LW, int BN = 128>
struct XDma {
    static constexpr int INS = BN * 17 / 64;
    static constexpr int NI = (INS + LW - 1) / LW;
    uint32_t off[NI]; // byte offset of the lane's (token, chunk) in the slice's x rows at stage 0
    int wv;
    __device__ void init(int64_t N, int64_t K, int64_t n0, int wv_, int lane) {
        wv = wv_;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int ins = min(wv + LW * i, INS - 1);
            const int slot = ins * 64 + lane, n = slot / 17, c = min(slot - 17 * n, 15);
            off[i] = 2 * ((uint32_t) (min<int64_t>(n0 + n, N - 1) * K) + 8 * c);
        }
    }
    // GA: the tile's tokens are the x rows rows[0 .. BN) (gathered pairs, repeated past the count)
    __device__ void init_rows(const int32_t * rows, int64_t K, int wv_, int lane) {
        wv = wv_;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int ins = min(wv + LW * i, INS - 1);
            const int slot = ins * 64 + lane, n = slot / 17, c = min(slot - 17 * n, 15);
            off[i] = 2 * ((uint32_t) rows[n] * (uint32_t) K + 8 * c);
        }
    }
    // the stage starting at element k0 into the LDS tile X
    __device__ void load(const uint16_t * xb, int k0, uint16_t * X) const {
        const uint8_t * base = reinterpret_cast<const uint8_t *>(xb) + 2 * (uint32_t) k0;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int ins = min(wv + LW * i, INS - 1);
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(base + off[i]),
                                             (__attribute__((address_space(3))) void *) (X + ins * 64 * 8), 16, 0, 0);
        }
    }
};

// The wide GEMM: one 12-wave work-group per CU as in the 12-wave k_matmul, but each wave owns 32
// weight rows x 128 tokens (NF = 4 token fragments), so every dequantized B fragment feeds 4 MFMAs
// instead of 2 (a 384-row x 128-token tile). NF = 2 (64 tokens) serves shapes with few tokens and
// many rows, bound by their weight stream. The dequantization VALU per MFMA halves; the
// registers for the extra accumulators come from the exact Q4_K form (s (c + bias) + o per pair,
// from plain x: no offset MFMA, no sub-block sums, no rare-scale branch), one set of A fragments
// (each read again right after the MFMA that consumed it), x tiles loaded straight into LDS and
// padded x rows (immediate LDS offsets). KG = 1: 12 row waves, 384-row tiles; KG = 2: 6 row
// waves x 2 groups that take half of K each (192-row tiles, for shapes the 384-row ones do not
// fill), each group finishing half of the token fragments; KG = 3 (64-token tiles): 4 row waves x
// 3 groups (128-row tiles), groups 1 and 2 handing their sums to group 0, which adds them in group
// order and stores. The 64-token forms also take the 64-token kernel's tile shapes wherever K is a
// whole number of stages, and GA runs the grouped MUL_MAT_ID (gathered x rows, scattered
// outputs). WV = 8 (KG = 1): 256-row tiles in 8-wave work-groups, one per CU (its LDS request
// keeps a second one off the CU), for shapes whose 384-row tiles leave CUs idle. Measured (quantized N(0, 0.02)
// weights): 12288 x 4096 at 2048 tokens 219 against 272 us, gate+up (24576 rows) at 512 tokens
// 118 against 145 us, 12288 x 4096 at 512 tokens (KG = 2) 70-76 against 79-82 us. Wave tiles of 64
// rows x 64 tokens (half the LDS reads per MFMA, twice the dequantization) measured slower than
// the 64-token form. Split-K over work-groups (partials + k_split_reduce) as in k_matmul.
template <int DT, int KG, int NF = 4, bool SK = false, bool GA = false, int WV = 12>
__global__ __launch_bounds__(64 * WV, 1) void k_gemm_w(MmArgs L) {
    constexpr int W = WV, BN = 32 * NF, RW = W / KG, BMT = 32 * RW;
    static_assert(W % KG == 0, "whole row waves per K group");
    static_assert(!SK || KG == 1, "stream-K runs 12 row waves");
    static_assert(!GA || (KG == 1 && !SK && NF == 2), "grouped MUL_MAT_ID: 384-row x 64-token tiles, no split");
    using F = PFmt<DT>;
    using Raw = typename F::Raw;
    extern __shared__ __attribute__((aligned(16))) uint16_t lds_mm[];
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // wave-uniform: scalar addressing
    const int wave = wid % RW, kg = wid / RW;                         // row wave, K group
    const int j = lane & 31, h = lane >> 5;
    // one piece of work: stages [p0, p1) of a tile. Split-K: the split's stages of tile
    // blockIdx.x / split. Stream-K: work-group g takes units [g U / G, (g + 1) U / G) of the
    // U = tiles x stages / 2 units of 2 stages (tile-major), at most two pieces since U / G is at
    // most a tile's units; a piece that is
    // not a whole tile stores its sums (x the rows' factors) into partial slot g + t, which
    // k_sk_reduce adds in work-group order (g + t rises by at least one from piece to piece, so
    // the slots are distinct)
    auto piece = [&](const int64_t tile, const int split, const int p0, const int p1, const int64_t slot) __attribute__((always_inline)) {
    const int64_t tm = tile % L.tiles_m, tn = tile / L.tiles_m;
    const int64_t sl = blockIdx.y;
    const int64_t i2 = sl % L.a.ne12, i3 = sl / L.a.ne12;
    const int64_t grow = tm * BMT + 32 * wave;
    const int mj = L.nmat == 1 ? 0
                 : L.packed    ? min(L.nmat - 1, grow >= L.mo[1] ? (grow >= L.mo[2] ? 2 : 1) : 0)
                               : (tm >= L.mt[1] ? (tm >= L.mt[2] ? 2 : 1) : 0);
    const uint8_t * w = L.nmat > 1 ? L.wm[mj] : L.a.w + (uint64_t) (i2 / L.a.r2) * L.a.w_s2 + (uint64_t) (i3 / L.a.r3) * L.a.w_s3;
    const int64_t K = L.a.K, nb = L.a.nb;
    int64_t N = L.a.N;
    const int64_t M = L.nmat > 1 ? L.Mm[mj] : L.a.M;
    int64_t n0 = tn * BN;
    const int64_t m0 = L.packed ? grow - L.mo[mj] : (tm - L.mt[mj]) * BMT + 32 * wave;
    // GA (grouped MUL_MAT_ID, as in k_matmul): token tile tn belongs to one expert, whose weights
    // the work-group reads; its tokens are gathered x rows and its outputs scattered through a
    // table in LDS after the x buffers
    int32_t * ga_rows = reinterpret_cast<int32_t *>(lds_mm + 2 * BN * XR); // x row of tile token n
    int64_t * ga_y = reinterpret_cast<int64_t *>(ga_rows + BN);           // its y element offset
    int32_t ga_cnt = BN;                                                  // the tile's pairs
    bool half_tile = false; // at most 32 pairs: the second token fragment is padding (wave-uniform)
    if constexpr (GA) {
        // the expert owning token tile tn: the last e with t_start[e] <= tn (an empty expert
        // shares its start with the next one)
        if (tn >= L.t_start[L.n_exp]) return; // past this call's tiles (the whole work-group)
        int lo = 0, hi = L.n_exp - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (L.t_start[mid] <= tn) lo = mid;
            else hi = mid - 1;
        }
        const int32_t pb = L.e_off[lo] + (int32_t) (tn - L.t_start[lo]) * BN;
        ga_cnt = min(BN, L.e_off[lo + 1] - pb);
        half_tile = ga_cnt <= 32;
        w = L.a.w + (uint64_t) lo * L.a.w_s2;
        if (threadIdx.x < BN) {
            const int32_t pr = L.pairs[pb + min((int) threadIdx.x, ga_cnt - 1)]; // tokens past the count repeat the last pair
            const int32_t t = pr / L.n_used, slot = pr - t * L.n_used;
            ga_rows[threadIdx.x] = t * L.x_cols + (L.x_cols > 1 ? slot : 0);
            ga_y[threadIdx.x] = (int64_t) slot * L.a.y_s1 + (int64_t) t * L.a.y_s2;
        }
        __syncthreads();
        N = BN;
        n0 = 0;
    }
    // the stages of the split (whole groups of 4) or of the K group (KG = 2: every group walks
    // 4 ceil(groups / 2) stages so that all waves meet the same barriers; a group's stages past K
    // are inactive: their loads repeat a valid stage, their k-steps are skipped), as in k_matmul
    const int64_t groups = (L.stages + 3) / 4;
    const int gsz = (int) (4 * ((groups + KG - 1) / KG));
    const int s0 = SK ? p0 : (int) (KG > 1 ? kg * gsz : 4 * (groups * split / L.split));
    const int s1 = SK ? p1 : (int) (KG > 1 ? min<int64_t>(s0 + gsz, L.stages) : min(4 * (groups * (split + 1) / L.split), L.stages));
    const int send = KG > 1 ? s0 + gsz : s1;
    const int lim = s1 - 1;

    F f;
    f.init(M, nb, RowAddr(M, m0 + j), h);
    const uint16_t * xb = L.xb + (uint64_t) sl * N * K;
    XDma<RW, BN> xt;
    if constexpr (GA) xt.init_rows(ga_rows, K, wave, lane);
    else xt.init(N, K, n0, wave, lane);
    uint16_t * const lds_x = lds_mm + kg * (2 * BN * XR); // the K group's two x buffers
    const int abase = j * XR; // + 32 q XR + 8 chunk(h, t): immediate offsets

    f32x16 acc[NF];
#pragma unroll
    for (int q = 0; q < NF; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[q][v] = 0.0f;

    // one stage: the weights of stage s + 1 into nw and its x tile into the other LDS buffer
    // (read by every wave before the last barrier) while the MFMAs run over buffer s % 2
    auto stage = [&](auto dtag, int s, const Raw & cw, Raw & nw) __attribute__((always_inline)) {
        constexpr int D = decltype(dtag)::value;
        const int sn = min(s + 1, lim);
        if constexpr ((DT == Q4_K || DT == Q6_K) && (D & 1) == 0) nw = f.load_half2(w, sn, cw);
        else nw = f.load(w, sn);
        if (s + 1 < s1) xt.load(xb, (s + 1) * BK, lds_x + ((D + 1) & 1) * (BN * XR));
        const uint16_t * X = lds_x + (D & 1) * (BN * XR) + abase;
        if (KG > 1 && s >= s1) { // an inactive stage (wave-uniform): only the barrier
            __syncthreads();
            return;
        }
        const typename F::Sc sc = f.prep(cw, (s & ~3) | D);
        f16x8 a[NF];
#pragma unroll
        for (int q = 0; q < NF; ++q) a[q] = *reinterpret_cast<const f16x8 *>(X + q * 32 * XR + 8 * F::chunk(h, 0));
        f16x8 b = F::bop(cw, sc, 0);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            // issue priority falling through the stage: the waves of a SIMD that are behind win
            // the arbitration, so they reach the stage barrier together
            if (t == 0) __builtin_amdgcn_s_setprio(3);
            if (t == 2) __builtin_amdgcn_s_setprio(2);
            if (t == 4) __builtin_amdgcn_s_setprio(1);
            if (t == 6) __builtin_amdgcn_s_setprio(0);
            f16x8 bn;
            if (t < 7) bn = F::bop(cw, sc, t + 1);
#pragma unroll
            for (int q = 0; q < NF; ++q) {
                if (!(GA && q > 0 && half_tile)) acc[q] = mma32<DT>(a[q], b, acc[q]);
                if (t < 7) a[q] = *reinterpret_cast<const f16x8 *>(X + q * 32 * XR + 8 * F::chunk(h, t + 1));
            }
            if (t < 7) b = bn;
        }
        __syncthreads(); // (waits for this wave's loads: the next x tile is in LDS)
    };
    Raw ra{}, rb{};
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    int s = s0;
    if constexpr (SK) {
        // a piece starts at an even stage: stages 2 and 3 of a group of 4 run first when it
        // starts inside one, tagged with their position in the unrolled group (LDS buffer,
        // half-block parity)
        ra = f.load(w, s0);
        xt.load(xb, s0 * BK, lds_x);
        __syncthreads();
        if (s0 & 2) {
            stage(I2{}, s, ra, rb);
            if (s + 1 < s1) stage(I3{}, s + 1, rb, ra);
            s += 2;
        }
    } else {
        ra = f.load(w, min(s0, lim));
        xt.load(xb, min(s0, lim) * BK, lds_x);
        __syncthreads();
    }
    for (; s + 3 < send; s += 4) {
        stage(I0{}, s, ra, rb);
        stage(I1{}, s + 1, rb, ra);
        stage(I2{}, s + 2, ra, rb);
        stage(I3{}, s + 3, rb, ra);
    }
    if (s < send) { // (KG = 2: send - s0 is a multiple of 4, no tail)
        stage(I0{}, s, ra, rb);
        if (s + 1 < s1) {
            stage(I1{}, s + 1, rb, ra);
            if (s + 2 < s1) stage(I2{}, s + 2, ra, rb);
        }
    }
    // acc[q][v], lane (j, h): token n0 + 32q + 8 (v / 4) + 4h + v % 4, weight row m0 + j
    auto store_out = [&](auto qb, auto qc) __attribute__((always_inline)) {
        constexpr int QB = decltype(qb)::value, QC = decltype(qc)::value;
        if constexpr (GA) {
            // scatter: token n of the tile is pair ga_y[n] (the pairs past ga_cnt are not stored)
            const int64_t m = m0 + j;
#pragma unroll
            for (int q = QB; q < QB + QC; ++q) {
                float u[16];
#pragma unroll
                for (int v = 0; v < 16; ++v) u[v] = L.xs[ga_rows[32 * q + 8 * (v >> 2) + 4 * h + (v & 3)]];
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int n = 32 * q + 8 * (v >> 2) + 4 * h + (v & 3);
                    if (n < ga_cnt && m < M) L.a.y[ga_y[n] + m] = acc[q][v] * u[v];
                }
            }
            return;
        }
        const int64_t slices = L.a.ne12 * L.a.ne13;
        float * y;
        int64_t ys1;
        int64_t m = m0 + j;
        if (SK && slot >= 0) { // a partial slot: [BN tokens][BMT rows] of the tile
            y = L.part + (uint64_t) slot * (BN * BMT) - n0 * BMT + 32 * wave + j - m;
            ys1 = BMT;
        } else if (L.split == 1) {
            y = L.nmat > 1 ? L.ym[mj] : L.a.y + i2 * L.a.y_s2 + i3 * L.a.y_s3;
            ys1 = L.nmat > 1 ? L.ys1m[mj] : L.a.y_s1;
        } else {
            const int64_t mt_all = L.mo[L.nmat];
            y = L.part + ((uint64_t) split * slices + (uint64_t) sl) * N * mt_all + L.mo[mj];
            ys1 = mt_all;
        }
        const float * xs = L.xs + (uint64_t) sl * N;
#pragma unroll
        for (int q = QB; q < QB + QC; ++q) {
            float u[16];
#pragma unroll
            for (int v = 0; v < 16; ++v) u[v] = xs[min<int64_t>(n0 + 32 * q + 8 * (v >> 2) + 4 * h + (v & 3), N - 1)];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t n = n0 + 32 * q + 8 * (v >> 2) + 4 * h + (v & 3);
                // (outputs are not read again by this kernel: stores that bypass the caches)
                if (n < N && m < M) __builtin_nontemporal_store(acc[q][v] * u[v], y + n * ys1 + m);
            }
        }
    };
    // KG = 2: each group finishes half of the token fragments, QB .. QB + QN: it hands the other
    // half of its sums to the other group through LDS (the x buffers are free now) and adds the
    // other group's half of its own (a + b = b + a exactly: no order to keep), so both groups store
    // KG = 3: groups 1 and 2 hand all their sums to group 0 through LDS, which adds them in group
    // order and stores every fragment
    constexpr int QN = KG == 3 ? NF : NF / KG;
    auto finish3 = [&]() __attribute__((always_inline)) {
        constexpr int PER = NF * 16;
        float * red = reinterpret_cast<float *>(lds_mm);
        __syncthreads();
        if (kg > 0) {
            float * r = red + ((size_t) ((kg - 1) * RW + wave) * PER) * 64 + lane;
#pragma unroll
            for (int q = 0; q < NF; ++q)
#pragma unroll
                for (int v = 0; v < 16; ++v) r[(q * 16 + v) * 64] = acc[q][v];
        }
        __syncthreads();
        if (kg == 0) {
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                const float * o = red + ((size_t) (g * RW + wave) * PER) * 64 + lane;
#pragma unroll
                for (int q = 0; q < NF; ++q)
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[q][v] += o[(q * 16 + v) * 64];
            }
            store_out(std::integral_constant<int, 0>{}, std::integral_constant<int, NF>{});
        }
    };
    auto finish = [&](auto gtag) __attribute__((always_inline)) {
        // (the group's fragments as a compile-time range: registers cannot be indexed at run time)
        constexpr int G = decltype(gtag)::value, QB = G * QN;
        if constexpr (KG > 1) {
            constexpr int PER = QN * 16, QO = (1 - G) * QN; // QO: the other group's fragments
            float * red = reinterpret_cast<float *>(lds_mm);
            __syncthreads();
            float * r = red + ((size_t) (G * RW + wave) * PER) * 64 + lane;
#pragma unroll
            for (int q = 0; q < QN; ++q)
#pragma unroll
                for (int v = 0; v < 16; ++v) r[(q * 16 + v) * 64] = acc[QO + q][v];
            __syncthreads();
            const float * o = red + ((size_t) ((1 - G) * RW + wave) * PER) * 64 + lane;
#pragma unroll
            for (int q = 0; q < QN; ++q)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[QB + q][v] += o[(q * 16 + v) * 64];
        }
        store_out(std::integral_constant<int, QB>{}, std::integral_constant<int, QN>{});
    };
    if constexpr (KG == 3) finish3();
    else if (KG == 1 || kg == 0) finish(std::integral_constant<int, 0>{});
    else finish(std::integral_constant<int, 1>{});
    };
    if constexpr (SK) {
        // units of 2 stages (the stage count is even)
        const int64_t S = L.stages / 2, U = L.tiles_m * L.tiles_n * S, G = gridDim.x, g = blockIdx.x;
        int64_t lo = g * U / G;
        const int64_t hi = (g + 1) * U / G;
        while (lo < hi) {
            const int64_t t = lo / S;
            const int p0 = (int) (lo - t * S), p1 = (int) min<int64_t>(S, hi - t * S);
            piece(t, 0, 2 * p0, 2 * p1, p0 == 0 && p1 == S ? -1 : g + t);
            lo = (t + 1) * S;
        }
    } else {
        piece(blockIdx.x / L.split, (int) (blockIdx.x % L.split), 0, 0, -1);
    }
}

// The narrow GEMM (9..128 tokens, up to ~2 R32 groups per CU): the tiled forms above spend such a
// shape on stage barriers, split-K partial sums and their reduce pass. Here a work-group owns RW
// R32 groups (32 weight rows each) over NF token fragments and the whole of K, KW waves per group
// taking consecutive runs of whole 2-stage units; the waves never meet until the end, where their
// sums are added pairwise in a fixed tree through LDS (deterministic) and stored with the rows'
// factors. A wave reads its A fragments straight from the fragment-ordered x (k_x_to_f16<..,
// FRAG>): one 16-byte load per lane is two 512-byte runs (the 32 tokens of the lane halves'
// chunks), kept in a ring 4 k-steps ahead of the MFMAs, and its weights one stage ahead, through
// the formats' exact dequantization (the wide GEMM's). With RW = 2 the waves of one K run read the
// same x at about the same time (the second mostly from L1). Grid: (work-groups of RW R32 groups
// of all matrices, slices, token fragments / NF): with few R32 groups, each group's fragments go
// to separate work-groups, gridDim.x apart in dispatch order (with the usual round-robin over the
// 8 XCDs and gridDim.x a multiple of 8, the same XCD, whose L2 serves the second reader of the
// weights). What bounds it: every wave reads 64 bytes of x per 18 bytes of Q4_K weights, so each
// CU moves ~1 MB of x from L2 per 12288x4096 op at 64 tokens (~80 GB/s per CU measured).
template <int DT, int NF, int KW, int RW = 1>
__global__ __launch_bounds__(64 * KW * RW) void k_gemm_n(MmArgs L) {
    using F = PFmt<DT>;
    using Raw = typename F::Raw;
    constexpr int RING = 4;
    extern __shared__ __attribute__((aligned(16))) float lds_n[]; // [RW][KW / 2][NF * 16][64]
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rw = wv % RW, kw = wv / RW;
    const int j = lane & 31, h = lane >> 5;
    // the wave's R32 group (past the last one: the last one again, not stored)
    const int64_t tm = min<int64_t>((int64_t) blockIdx.x * RW + rw, L.tiles_m - 1), sl = blockIdx.y;
    const bool live = (int64_t) blockIdx.x * RW + rw < L.tiles_m;
    const int64_t i2 = sl % L.a.ne12, i3 = sl / L.a.ne12;
    const int mj = L.nmat == 1 ? 0 : (tm >= L.mt[1] ? (tm >= L.mt[2] ? 2 : 1) : 0);
    const uint8_t * w = L.nmat > 1 ? L.wm[mj] : L.a.w + (uint64_t) (i2 / L.a.r2) * L.a.w_s2 + (uint64_t) (i3 / L.a.r3) * L.a.w_s3;
    const int64_t nb = L.a.nb, N = L.a.N;
    const int64_t M = L.nmat > 1 ? L.Mm[mj] : L.a.M;
    const int64_t m0 = (tm - L.mt[mj]) * 32;
    const int S = (int) L.stages, U = (S + 1) / 2; // units of 2 stages (the K-quants' blocks)
    const int s0 = 2 * (U * kw / KW), s1 = min(2 * (U * (kw + 1) / KW), S), lim = max(s1 - 1, 0);

    F f;
    f.init(M, nb, RowAddr(M, m0 + j), h);
    // x fragment (q, stage s, k-step t): 16 bytes at xq + (q S + s) 8192 + co[t]
    const int tf = (int) ((N + 31) / 32);                // the slice's token fragments
    const int qz = (int) blockIdx.z * NF;                // this work-group's first one
    const uint8_t * xq = reinterpret_cast<const uint8_t *>(L.xb) + ((uint64_t) sl * tf + qz) * S * 8192;
    uint32_t co[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) co[t] = (uint32_t) (F::chunk(h, t) * 32 + j) * 16;
    auto xload = [&](int s, int t, int q) __attribute__((always_inline)) {
        return *reinterpret_cast<const f16x8 *>(xq + ((uint32_t) (q * S + s) * 8192u + co[t]));
    };

    f32x16 acc[NF];
#pragma unroll
    for (int q = 0; q < NF; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[q][v] = 0.0f;

    if (s0 < s1) { // (wave-uniform: K shorter than a unit per wave leaves some waves idle)
        f16x8 ring[RING][NF];
        // one stage: the weights of stage s + 1 into nw; k-step t's A fragments come from the ring,
        // which takes k-step t + 4 (of this stage or the next) in their place
        auto stage = [&](auto dtag, int s, const Raw & cw, Raw & nw) __attribute__((always_inline)) {
            constexpr int D = decltype(dtag)::value;
            const int sn = min(s + 1, lim);
            if constexpr ((DT == Q4_K || DT == Q6_K) && D == 0) nw = f.load_half2(w, sn, cw);
            else nw = f.load(w, sn);
            // (the loads stay where they are issued: the scheduler would sink them to their use)
            __builtin_amdgcn_sched_barrier(0);
            const typename F::Sc sc = f.prep(cw, (s & ~1) | D);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const f16x8 b = F::bop(cw, sc, t);
                f16x8 a[NF];
#pragma unroll
                for (int q = 0; q < NF; ++q) {
                    a[q] = ring[t % RING][q];
                    ring[t % RING][q] = t + RING < 8 ? xload(s, t + RING, q) : xload(sn, t + RING - 8, q);
                }
#pragma unroll
                for (int q = 0; q < NF; ++q) acc[q] = mma32<DT>(a[q], b, acc[q]);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        Raw ra = f.load(w, s0), rb;
#pragma unroll
        for (int t = 0; t < RING; ++t)
#pragma unroll
            for (int q = 0; q < NF; ++q) ring[t][q] = xload(s0, t, q);
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        // (no stage under a branch inside the loop: the compiler would then wait for every load in
        // flight at the loop's head)
        int s = s0;
        for (; s + 1 < s1; s += 2) {
            stage(I0{}, s, ra, rb);
            stage(I1{}, s + 1, rb, ra);
        }
        if (s < s1) stage(I0{}, s, ra, rb); // (an odd stage count: Q4_0 / Q8_0 only)
    }
    // the waves' sums, pairwise in a fixed tree (deterministic): in round r waves r .. 2r - 1 hand
    // theirs through LDS to waves 0 .. r - 1, which add them; wave 0 stores. acc[q][v], lane (j, h):
    // token 32 q + 8 (v / 4) + 4 h + v % 4, weight row m0 + j
    constexpr int PER = NF * 16 * 64;
#pragma unroll
    for (int r = KW / 2; r >= 1; r /= 2) {
        if (kw >= r && kw < 2 * r) {
#pragma unroll
            for (int q = 0; q < NF; ++q)
#pragma unroll
                for (int v = 0; v < 16; ++v) lds_n[(rw * (KW / 2) + kw - r) * PER + (q * 16 + v) * 64 + lane] = acc[q][v];
        }
        __syncthreads();
        if (kw < r) {
#pragma unroll
            for (int q = 0; q < NF; ++q)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[q][v] += lds_n[(rw * (KW / 2) + kw) * PER + (q * 16 + v) * 64 + lane];
        }
        if (r > 1) __syncthreads();
    }
    if (kw != 0 || !live) return;
    float * y = L.nmat > 1 ? L.ym[mj] : L.a.y + i2 * L.a.y_s2 + i3 * L.a.y_s3;
    const int64_t ys1 = L.nmat > 1 ? L.ys1m[mj] : L.a.y_s1;
    const float * xs = L.xs + (uint64_t) sl * N;
    const int64_t m = m0 + j;
#pragma unroll
    for (int q = 0; q < NF; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t n = 32 * (qz + q) + 8 * (v >> 2) + 4 * h + (v & 3);
            if (n < N && m < M) y[n * ys1 + m] = acc[q][v] * xs[n];
        }
}

// y = sum of the split-K partials, in split order. blockIdx.x is the row (token n of slice sl),
// blockIdx.y covers 1024 columns of it (all matrices' rows when several share x; column c is row
// c - mo[j] of matrix j); VEC when every matrix's rows and y's row starts allow float4 accesses.
template <bool VEC>
__global__ __launch_bounds__(256) void k_split_reduce(MmArgs L) {
    const int64_t N = L.a.N, Mt = L.mo[L.nmat];
    const int64_t row = blockIdx.x, sl = row / N, n = row - sl * N;
    const int64_t i2 = sl % L.a.ne12, i3 = sl / L.a.ne12;
    const uint64_t plane = (uint64_t) L.a.ne12 * L.a.ne13 * N * Mt;
    const float * p = L.part + row * Mt;
    auto out = [&](int64_t c) -> float * { // y element of column c
        const int j = c >= L.mo[1] ? (c >= L.mo[2] ? 2 : 1) : 0;
        float * y = L.nmat > 1 ? L.ym[j] + n * L.ys1m[j] : L.a.y + i2 * L.a.y_s2 + i3 * L.a.y_s3 + n * L.a.y_s1;
        return y + (c - L.mo[j]);
    };
    const int64_t m = ((int64_t) blockIdx.y * 256 + threadIdx.x) * 4;
    if (VEC) {
        if (m >= Mt) return;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int sp = 0; sp < L.split; ++sp) {
            const float4 u = *reinterpret_cast<const float4 *>(p + sp * plane + m);
            v.x += u.x;
            v.y += u.y;
            v.z += u.z;
            v.w += u.w;
        }
        *reinterpret_cast<float4 *>(out(m)) = v;
    } else {
        for (int64_t e = m; e < m + 4 && e < Mt; ++e) {
            float v = 0.0f;
            for (int sp = 0; sp < L.split; ++sp) v += p[sp * plane + e];
            *out(e) = v;
        }
    }
}

// stream-K: y = the sum of a tile's partial slots in work-group order, for the tiles that more
// than one work-group shared (k_gemm_w<.., SK>). blockIdx.x is the tile, blockIdx.y covers 1024
// of its BN x 384 sums (4 consecutive rows of one token per thread); VEC when every matrix's rows
// and y's rows allow float4 stores. One slice.
template <bool VEC, int BN = 128>
__global__ __launch_bounds__(256) void k_sk_reduce(MmArgs L) {
    constexpr int BMT = 384, TE = BN * BMT;
    const int64_t S = L.stages / 2, U = L.tiles_m * L.tiles_n * S, G = L.sk_g, t = blockIdx.x; // (units of 2 stages)
    // the work-groups g with g U / G <= t S < (g + 1) U / G, and with (t + 1) S - 1 in their range
    const int64_t ga = ((t * S + 1) * G + U - 1) / U - 1, gb = ((t + 1) * S * G + U - 1) / U - 1;
    if (ga == gb) return; // a whole tile of one work-group: stored by it
    const int e = (blockIdx.y * 256 + threadIdx.x) * 4;
    if (e >= TE) return;
    const int nl = e / BMT, ml = e - nl * BMT;
    const int64_t tm = t % L.tiles_m, n = t / L.tiles_m * BN + nl;
    if (n >= L.a.N) return;
    int mj = 0;
    int64_t m = tm * BMT + ml;
    if (L.nmat > 1) {
        if (L.packed) {
            mj = min(L.nmat - 1, m >= L.mo[1] ? (m >= L.mo[2] ? 2 : 1) : 0);
            m -= L.mo[mj];
        } else {
            mj = tm >= L.mt[1] ? (tm >= L.mt[2] ? 2 : 1) : 0;
            m = (tm - L.mt[mj]) * BMT + ml;
        }
    }
    const int64_t M = L.nmat > 1 ? L.Mm[mj] : L.a.M;
    if (m >= M) return;
    float * y = (L.nmat > 1 ? L.ym[mj] + n * L.ys1m[mj] : L.a.y + n * L.a.y_s1) + m;
    const float * p = L.part + (uint64_t) (ga + t) * TE + e;
    // up to 8 slots loaded together, then added in order
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int64_t g0 = 0; g0 <= gb - ga; g0 += 8) {
        float4 u[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (g0 + i <= gb - ga) u[i] = *reinterpret_cast<const float4 *>(p + (uint64_t) (g0 + i) * TE);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (g0 + i <= gb - ga) {
                v.x += u[i].x;
                v.y += u[i].y;
                v.z += u[i].z;
                v.w += u[i].w;
            }
    }
    if (VEC) {
        *reinterpret_cast<float4 *>(y) = v;
    } else {
        const float r[4] = {v.x, v.y, v.z, v.w};
        for (int i = 0; i < 4 && m + i < M; ++i) y[i] = r[i];
    }
}

// x (f32, strided rows) -> f16 rows of K contiguous elements, one work-group per row (token n of
// slice sl = blockIdx.x / N). The row is scaled by 2^e so that its largest magnitude lands in
// [2^14, 2^15): no row overflows f16 and none loses precision to its subnormals beyond 2^-24 of
// the row's maximum; xs[row] = 2^-e undoes it on the products. Inside each group of 4 elements the
// order is 0 2 1 3, the order of the weight pairs the matmul builds. VEC: rows 16-byte aligned.
// The first kCached groups of 8 elements per thread stay in registers between the two passes.
// Q4K (the single-fma weight form): elements 32..63 of every 64 (the high nibbles of a Q4_K group)
// are stored divided by 16 more, and xsum gets the row's 32-element sub-block sums (of the scaled
// x, times 1/32 so that they fit f16), 16 per 512 elements in the order the matmul's lanes hold
// the sub-blocks: position 8 h + e <- sub-block 4 (e / 2) + 2 h + e % 2; missing ones are zero.
// FRAG (K a multiple of the 128-element stage): the rows in the order the narrow GEMM reads them,
// chunk c (8 elements) of stage s of token n at ((n / 32 * stages + s) * 16 + c) * 32 + n % 32 in
// units of 16 bytes (per slice, tokens padded to a multiple of 32): the 32 tokens of one chunk
// are 512 contiguous bytes.
// (tid: the thread's index among the row's 256, wmax: 4 floats of LDS for the row's waves; a
// thread group with live = false takes part in the barrier only)
template <bool VEC, bool Q4K, bool BF, bool FRAG>
__device__ __forceinline__ void x_row_to_f16(const MatArgs & a, uint16_t * xb, float * xs, uint16_t * xsum, int64_t xsum_row, int64_t row,
                                             int tid, float * wmax, bool live) {
    constexpr int kCached = 6; // K <= 12288 is read once
    const int64_t sl = row / a.N, n = row - sl * a.N;
    const int64_t i2 = sl % a.ne12, i3 = sl / a.ne12;
    const float * xp = a.x + i2 * a.x_s2 + i3 * a.x_s3 + n * a.x_s1;
    uint16_t * op = xb + row * a.K;
    if constexpr (FRAG)
        op = xb + ((sl * ((a.N + 31) / 32) + n / 32) * (a.K / BK) * kChunks * 32 + n % 32) * 8;
    auto load8 = [&](int64_t k, float * v) {
        if (VEC) {
            const float4 u = *reinterpret_cast<const float4 *>(xp + k);
            const float4 t = *reinterpret_cast<const float4 *>(xp + k + 4);
            v[0] = u.x, v[1] = u.y, v[2] = u.z, v[3] = u.w, v[4] = t.x, v[5] = t.y, v[6] = t.z, v[7] = t.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = xp[k + e];
        }
    };
    auto store8 = [&](int64_t k, const float * v, int e2) {
        float s[8];
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            s[e] = ldexpf(v[e], e2);
            sum += s[e];
        }
        if constexpr (Q4K) {
            // the 4 threads of a 32-element sub-block are lanes 4m .. 4m + 3 of one wave
            sum += __shfl_xor(sum, 1);
            sum += __shfl_xor(sum, 2);
            if ((tid & 3) == 0 && live) {
                const int64_t jb = k >> 5, jj = jb & 15;
                const int64_t pos = (jb >> 4) * 16 + 8 * ((jj >> 1) & 1) + 2 * (jj >> 2) + (jj & 1);
                xsum[row * xsum_row + pos] = __half_as_ushort(__float2half(sum * 0.03125f));
            }
            if (k & 32) {
#pragma unroll
                for (int e = 0; e < 8; ++e) s[e] *= 0.0625f;
            }
        }
        if (!live) return;
        if constexpr (BF) { // (BF16 weights: x in bf16, rounded to nearest even)
            const bf16x2 p0 = __builtin_convertvector((f32x2{s[0], s[2]}), bf16x2), p1 = __builtin_convertvector((f32x2{s[1], s[3]}), bf16x2);
            const bf16x2 p2 = __builtin_convertvector((f32x2{s[4], s[6]}), bf16x2), p3 = __builtin_convertvector((f32x2{s[5], s[7]}), bf16x2);
            *reinterpret_cast<uint4 *>(op + k) = make_uint4(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                                                            __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3));
        } else {
            const f16x2 p0 = __builtin_convertvector((f32x2{s[0], s[2]}), f16x2), p1 = __builtin_convertvector((f32x2{s[1], s[3]}), f16x2);
            const f16x2 p2 = __builtin_convertvector((f32x2{s[4], s[6]}), f16x2), p3 = __builtin_convertvector((f32x2{s[5], s[7]}), f16x2);
            // (FRAG: chunk k / 8 of the row is chunk k / 8 % 16 of stage k / 128)
            uint16_t * d = FRAG ? op + ((k >> 7) * kChunks * 32 + ((k >> 3) & 15) * 32) * 8 : op + k;
            *reinterpret_cast<uint4 *>(d) = make_uint4(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                                                       __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3));
        }
    };
    const int64_t k0 = (int64_t) tid * 8; // K is a multiple of 32: a group of 8 is whole
    float cache[kCached][8];
    float mx = 0.0f;
#pragma unroll
    for (int c = 0; c < kCached; ++c) {
        const int64_t k = k0 + (int64_t) c * 2048;
        if (k < a.K) {
            load8(k, cache[c]);
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(cache[c][e]));
        }
    }
    for (int64_t k = k0 + (int64_t) kCached * 2048; k < a.K; k += 2048) {
        float v[8];
        load8(k, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[e]));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((tid & 63) == 0) wmax[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int e2 = 0;
    if (mx > 0.0f && mx <= 3.4e38f) {
        int ex;
        frexpf(mx, &ex); // mx = f 2^ex, f in [0.5, 1)
        e2 = min(15 - ex, 120);
    }
    if (tid == 0 && live) xs[row] = ldexpf(1.0f, -e2);
#pragma unroll
    for (int c = 0; c < kCached; ++c) {
        const int64_t k = k0 + (int64_t) c * 2048;
        if (k < a.K) store8(k, cache[c], e2);
    }
    for (int64_t k = k0 + (int64_t) kCached * 2048; k < a.K; k += 2048) {
        float v[8];
        load8(k, v);
        store8(k, v, e2);
    }
    if constexpr (Q4K) {
        for (int64_t jb = a.K / 32 + tid; live && jb < xsum_row; jb += 256) {
            const int64_t jj = jb & 15;
            xsum[row * xsum_row + (jb >> 4) * 16 + 8 * ((jj >> 1) & 1) + 2 * (jj >> 2) + (jj & 1)] = 0;
        }
    }
}

template <bool VEC, bool Q4K, bool BF = false, bool FRAG = false>
__global__ __launch_bounds__(256) void k_x_to_f16(MatArgs a, uint16_t * xb, float * xs, uint16_t * xsum, int64_t xsum_row) {
    __shared__ float wmax[4];
    x_row_to_f16<VEC, Q4K, BF, FRAG>(a, xb, xs, xsum, xsum_row, blockIdx.x, threadIdx.x, wmax, true);
}

// MUL_MAT_ID routing (E <= 1024 experts, P < 2^24 pairs), by one 1024-thread work-group: the
// pairs p = t * n_used + slot grouped by expert (ids clamped to [0, E)); e_off[e] / t_start[e] =
// the first pair / token tile (bn pairs) of expert e, [E] = the totals. Counts with LDS atomics,
// exclusive scans of the counts and of the tile counts (one expert per thread, wave scans), then
// each pair placed at its expert's cursor (its id read again: it is in the L2 by then). The order
// of the pairs inside an expert follows the LDS atomics; no output depends on it (each is one
// pair's own sum over K).
struct RouteArgs {
    const int32_t * ids;
    int64_t s0, s1;
    int nu, T, E, bn;
    int32_t * e_off;
    int32_t * t_start;
    int32_t * pairs;
};

__device__ __forceinline__ void moe_route(const RouteArgs & r) {
    __shared__ int32_t cnt[1024], cur[1024], wsum[2][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int P = r.nu * r.T;
    auto expert = [&](int p) {
        const int t = p / r.nu, slot = p - t * r.nu;
        return min(max(r.ids[slot * r.s0 + t * r.s1], 0), r.E - 1);
    };
    cnt[tid] = 0;
    __syncthreads();
    for (int p = tid; p < P; p += 1024) atomicAdd(&cnt[expert(p)], 1);
    __syncthreads();
    const int c = tid < r.E ? cnt[tid] : 0;
    const int tl = (c + r.bn - 1) / r.bn;
    int a = c, b = tl;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int ua = __shfl_up(a, o), ub = __shfl_up(b, o);
        if (lane >= o) {
            a += ua;
            b += ub;
        }
    }
    if (lane == 63) {
        wsum[0][wave] = a;
        wsum[1][wave] = b;
    }
    __syncthreads();
    int ea = a - c, eb = b - tl; // exclusive prefixes
    for (int w2 = 0; w2 < wave; ++w2) {
        ea += wsum[0][w2];
        eb += wsum[1][w2];
    }
    if (tid < r.E) {
        r.e_off[tid] = ea;
        r.t_start[tid] = eb;
        cur[tid] = ea;
    }
    if (tid == r.E - 1) {
        r.e_off[r.E] = ea + c;
        r.t_start[r.E] = eb + tl;
    }
    __syncthreads();
    for (int p = tid; p < P; p += 1024) r.pairs[atomicAdd(&cur[expert(p)], 1)] = p;
}

// the grouped MUL_MAT_ID's first launch: work-group 0 routes the pairs while the others convert
// the x rows, 4 per work-group (k_x_to_f16's work, rows 4 (blockIdx.x - 1) + threadIdx.x / 256):
// the routing's round trips run beside the conversion instead of in a launch of their own
template <bool VEC, bool Q4K>
__global__ __launch_bounds__(1024) void k_x_route(MatArgs a, uint16_t * xb, float * xs, uint16_t * xsum, int64_t xsum_row, int64_t rows,
                                                  RouteArgs r) {
    if (blockIdx.x == 0) {
        moe_route(r);
        return;
    }
    __shared__ float wmax[16];
    const int q = threadIdx.x >> 8;
    const int64_t row = 4 * ((int64_t) blockIdx.x - 1) + q;
    const bool live = row < rows;
    x_row_to_f16<VEC, Q4K, false, false>(a, xb, xs, xsum, xsum_row, live ? row : 0, threadIdx.x & 255, wmax + 4 * q, live);
}

int env_int(const char * name, int dflt) {
    const char * v = std::getenv(name);
    return v != nullptr && *v ? std::atoi(v) : dflt;
}

// Tile shape and work-groups along K per tile. A work-group is 4 waves; each wave owns RG groups
// of 32 weight rows (the tile is 128 RG rows) and BN tokens. Every A fragment read from LDS feeds
// RG MFMAs. Splits along K are added while the tiles leave the CUs' work-group slots empty, each
// split keeping >= 8 stages of K.
struct MmConfig {
    int bn, rg;
    int split;
    int w;  // waves per work-group: 4, or 12 (one work-group per CU, see k_matmul), or 8 (the wide GEMM's 256-row tiles)
    int kg; // K groups of a 12-wave work-group: 1 or 3
    bool wide = false; // k_gemm_w (w = 12): 128-token wave tiles (kg 1 or 2, bn = 128), or 64-token ones (kg = 1, bn = 64); w = 8: 256-row x 128-token tiles
    bool sk = false;   // the wide form's stream-K (kg = 1, bn = 128): cu_count work-groups share all tiles' stages
    bool narrow = false; // k_gemm_n: 9..128 tokens, rw R32 groups per work-group, kw waves along K each
    int kw = 8;
    int nz = 1; // narrow: work-groups per R32 group, each with bn / nz tokens
    int rw = 1; // narrow: R32 groups per work-group (kw waves each)
};

// the narrow GEMM's shapes: quantized weights, 9..128 tokens, one slice, K a whole number of
// stages; x then goes to scratch in fragment order, its token rows padded to a multiple of 32
bool narrow_shape(const MatArgs & a) {
    static const int env = env_int("SCRAPGPU_HIP_MM_NARROW", 1);
    return env != 0 && (a.dtype == Q4_0 || a.dtype == Q8_0 || a.dtype == Q4_K || a.dtype == Q6_K) && a.N > 8 && a.N <= 128 &&
           a.ne12 * a.ne13 == 1 && a.K % BK == 0;
}


MmConfig config_of(const MatArgs & a, int cu_count, bool lean) {
    static const int env_bn = env_int("SCRAPGPU_HIP_MM_BN", 0), env_rg = env_int("SCRAPGPU_HIP_MM_RG", 0);
    static const int env_split = env_int("SCRAPGPU_HIP_MM_SPLIT", 0);
    const int64_t slices = a.ne12 * a.ne13;
    const int64_t stages = (a.K + BK - 1) / BK;
    static const int env_w = env_int("SCRAPGPU_HIP_MM_W", 0);
    MmConfig c;
    if (narrow_shape(a) && env_w == 0 && env_bn == 0 && env_split == 0) {
        static const int env_kw = env_int("SCRAPGPU_HIP_MM_KW", 0);
        // R32 groups < CUs: one group per work-group (and 64 tokens as two work-groups of 32,
        // 8 waves each; 32 tokens in 16 waves); up to 2x the CUs: two groups per work-group (the
        // waves of a K run read the same x, the second mostly from L1). Measured on 256 CUs
        // (op time with the x pre-pass, against the forms below): Q4_K 12288x4096 at 64 / 32 / 16
        // tokens 26.8 / 19.9 / 18.9 against 31.4 / 27.6 / 26.5 us, 4096x12288 at 64 / 32 27.9 /
        // 25.2 against 31.1 / 28.9, 4096x4096 at 64 16.2 against 23.2; more groups lost (gate+up
        // 24576 rows 38-39 against 35.6, the Q6_K LM head 224-246 against 153)
        static const int env_nz = env_int("SCRAPGPU_HIP_MM_NZ", 0);
        static const int env_rw = env_int("SCRAPGPU_HIP_MM_RW", 0);
        const int64_t groups = (a.M + 31) / 32;
        // (65..128 tokens: two work-groups of 64 per R32 group where the groups are fewer than the
        // CUs: 4096x4096 22.4 against 32.2 us, 6144x4096 28.1 against 34.7, 4096x12288 38.9 against
        // 41.4; 12288x4096 lost, 41.1 against 36.0)
        // 33..128 tokens where 3 R32 groups per work-group, the tokens in two halves (two
        // work-groups per triple of groups, gridDim.x apart), fill the CUs in one round (15/16 of
        // them or more): 12 waves, 4 along K per group. 12288x4096 at 64 tokens 26.0 -> 23.5 us
        // against 2 groups per work-group (192 work-groups), Q6_K 28.1 -> 26.2, at 48 tokens 25.5 ->
        // 23.7; at 128 tokens 35.1 against 35.7-36.0 for the wide GEMM's 64-token tiles
        const int64_t t3 = (groups + 2) / 3 * 2;
        const bool fill3 = a.N > 32 && t3 <= cu_count && 16 * t3 >= 15 * (int64_t) cu_count;
        if ((a.N <= 64 ? groups <= 2 * (int64_t) cu_count : groups < cu_count) || (env_rw == 0 && fill3) || env_rw > 0) {
            c.narrow = true;
            c.kg = c.rg = c.split = 1;
            c.bn = a.N <= 32 ? 32 : a.N <= 64 ? 64 : 128;
            c.rw = env_rw == 1 || env_rw == 2 || env_rw == 3 || env_rw == 4 ? env_rw : fill3 ? 3 : groups < cu_count ? 1 : 2;
            c.nz = c.rw == 1 && c.bn == 64 && (env_nz == 2 || (env_nz == 0 && groups < cu_count)) ? 2 : 1;
            if (c.bn == 128) c.nz = env_nz == 4 && c.rw == 1 ? 4 : 2;
            if (c.rw == 3) {
                if (c.bn == 32) c.rw = 2; // (not built: 32 tokens would leave a third of the work-groups)
                else {
                    c.nz = 2;
                    c.kw = 4;
                    c.w = 12;
                    return c;
                }
            }
            if (c.rw == 1) {
                c.kw = env_kw == 8 || env_kw == 16 ? env_kw : groups * c.nz >= cu_count ? 8 : 16;
                if (c.kw == 16 && c.bn / c.nz == 64) c.kw = 8; // (64 tokens in 16 waves: more registers than 1024 threads allow)
            } else {
                if (c.rw == 4 && c.bn / c.nz == 64) c.rw = 2; // (not built)
                c.kw = c.bn / c.nz == 64 || c.rw == 4 ? 4 : 8;
            }
            c.w = c.kw * c.rw;
            return c;
        }
    }
    if (a.dtype == F16 || a.dtype == BF16) {
        // the wide GEMM (k_gemm_w, 384-row x 128-token tiles; its 2-K-group form spills with the
        // float rows' raw data) where its tiles fill the CUs, or with K split so that they occupy
        // 2/3 of them or more in one round, >= 16 stages per split
        static const int env_wide = env_int("SCRAPGPU_HIP_MM_WIDE", 1);
        if (env_wide != 0 && env_w == 0 && env_bn == 0 && env_split <= 1 && a.K % BK == 0 && a.N >= 128 &&
            (a.N + 127) / 128 * 128 * 8 <= 9 * a.N && (a.M % 384 == 0 || a.M >= 8 * 384)) {
            const int64_t tw = (a.M + 383) / 384 * ((a.N + 127) / 128) * slices;
            c.w = 12;
            c.kg = 1;
            c.rg = 1;
            c.bn = 128;
            c.wide = true;
            c.split = 1;
            if (tw % cu_count == 0 || tw >= 4 * (int64_t) cu_count) return c;
            if (slices == 1) // (at most 2 splits: 3 and 4 measured slower than the 4-wave form)
                for (int sp = 2; sp <= 2; ++sp)
                    if (tw * sp <= cu_count && 3 * tw * sp >= 2 * cu_count && stages / sp >= 16) {
                        c.split = sp;
                        return c;
                    }
            c.wide = false;
        }
        // else 4-wave work-groups, 128-token tiles from 128 tokens on (each 2-byte weight fetched
        // half as often: 12288x4096 at 512 tokens 119 against 137 us, at 256 tokens 81 against 92)
        c.w = 4;
        c.kg = 1;
        c.rg = 1;
        const int64_t tm = (a.M + 127) / 128;
        c.bn = env_bn == 64 || env_bn == 128 ? env_bn : a.N >= 128 ? 128 : 64;
        const int64_t tiles = tm * ((a.N + c.bn - 1) / c.bn) * slices;
        // the split with the least estimated time: rounds of cu_count work-groups x (stages per
        // split + 4, a work-group's fixed cost in stages), the fewer splits on a tie, every split
        // >= 8 stages (F16, 128-token tiles, measured on 256 CUs: 12288x4096 at 128 tokens, 96
        // tiles, 55.7 / 64.6 / 56.3 / 62.4 us at 2 / 3 / 4 / 8 splits; 4096x4096, 32 tiles, 31 us
        // at 8 against 36 at 4; 12288x4096 at 256 tokens 78 us unsplit against 80-87 split)
        c.split = 1;
        if (env_split > 0) {
            c.split = (int) std::max<int64_t>(1, std::min<int64_t>(std::min(env_split, 8), (stages + 3) / 4));
            return c;
        }
        auto cost = [&](int sp) { return (tiles * sp + cu_count - 1) / cu_count * ((stages + sp - 1) / sp + 4); };
        for (int sp = 2; sp <= 8 && stages / sp >= 8; ++sp)
            if (cost(sp) < cost(c.split)) c.split = sp;
        return c;
    }
    // 12-wave work-groups, one per CU, in this order of preference:
    //  1. KG = 1: 384-row tiles of 64 tokens that fill the CUs in whole rounds (or in enough
    //     rounds that the last one matters little), the last row tile mostly inside M;
    //  2. KG = 2: 192-row tiles that fill them, K in two equal runs of whole groups of 4 stages;
    //  3. KG = 3: 128-row tiles that fill them, K in three such runs (the groups take
    //     4 ceil(stages / 12) stages each; the last one's inactive stages, at most an eighth of
    //     the work, wait at the barriers);
    //  4. KG = 1 with K split over 2..4 work-groups (partial sums in HBM, then k_split_reduce)
    //     when that makes the 384-row tiles fill them, every split at least 8 stages.
    {
        static const int env_kg = env_int("SCRAPGPU_HIP_MM_KG", 0);
        const bool free_choice = env_w == 0 && env_bn != 128 && env_rg != 2 && env_split <= 1;
        auto fill = [&](int64_t t) { return t % cu_count == 0 || t >= 4 * (int64_t) cu_count; };
        const int64_t nt = (a.N + 63) / 64 * slices;
        const int64_t t12 = (a.M + 383) / 384 * nt, t6 = (a.M + 191) / 192 * nt, t4 = (a.M + 127) / 128 * nt;
        int s12 = 0;
        if (a.M % 384 == 0 || a.M >= 8 * 384)
            for (int sp = 1; sp <= 4 && s12 == 0; ++sp)
                if (fill(t12 * sp) && (sp == 1 || stages / sp >= 8)) s12 = sp;
        const int64_t gsz2 = 4 * (((stages + 3) / 4 + 1) / 2), gsz3 = 4 * (((stages + 3) / 4 + 2) / 3);
        const bool fits2 = fill(t6) && (a.M % 192 == 0 || a.M >= 8 * 192) && stages >= 16 && (2 * gsz2 - stages) * 8 <= stages;
        const bool fits3 = fill(t4) && stages >= 24 && (3 * gsz3 - stages) * 8 <= stages;
        c.w = 12;
        c.bn = 64;
        c.rg = 1;
        c.split = 1;
        // the wide form first (k_gemm_w): 128-token tiles (at most an eighth of the token tiles
        // padding) of 384 rows that fill the CUs, or of 192 rows with K in two equal runs of whole
        // groups of 4 stages; K a whole number of stages (its x tiles are loaded without a K tail)
        static const int env_wide = env_int("SCRAPGPU_HIP_MM_WIDE", 1);
        if (env_wide != 0 && free_choice && env_kg != 3 && a.K % BK == 0 && a.N >= 128 && (a.N + 127) / 128 * 128 * 8 <= 9 * a.N) {
            const int64_t ntw = (a.N + 127) / 128 * slices;
            c.bn = 128;
            c.wide = true;
            if (env_kg != 2 && (a.M % 384 == 0 || a.M >= 8 * 384) && fill((a.M + 383) / 384 * ntw)) {
                c.kg = 1;
                return c;
            }
            if (env_kg != 1 && (a.M % 192 == 0 || a.M >= 8 * 192) && fill((a.M + 191) / 192 * ntw) && stages >= 16 && (2 * gsz2 - stages) * 8 <= stages) {
                c.kg = 2;
                return c;
            }
            // 8-wave work-groups of 256-row x 128-token tiles, one per CU, with K split over sp of
            // them, where that fills the CUs in one round (at least 15/16 of them) with >= 16
            // stages per split: fewer waves per CU than the 12-wave forms, but every CU at work
            // (4096x12288 at 512 tokens: 64 tiles x 4 splits, 75.6 against 85.3 us per op for 44
            // 384-row tiles x 4 splits; Q6_K 78.2 against 87.5, Q8_0 4096x11008 77.1 against 86.4;
            // at 2048 tokens 256 tiles unsplit, 232-237 against 257-262 for stream-K; at 1024
            // tokens 128 x 2, 128.6 against 140.3)
            static const int env_w8 = env_int("SCRAPGPU_HIP_MM_W8", 1);
            if (env_w8 != 0 && env_kg != 2 && slices == 1 && (a.M % 256 == 0 || a.M >= 8 * 256)) {
                const int64_t t8 = (a.M + 255) / 256 * ntw;
                for (int sp = 1; sp <= 8; ++sp)
                    if (t8 * sp <= cu_count && 16 * t8 * sp >= 15 * (int64_t) cu_count && stages / sp >= 16) {
                        c.w = 8;
                        c.kg = 1;
                        c.split = sp;
                        return c;
                    }
            }
            static const int env_ws = env_int("SCRAPGPU_HIP_MM_WSPLIT", 0);
            if (env_ws > 1) {
                c.kg = env_kg == 2 ? 2 : 1;
                if (c.kg == 1) c.split = env_ws;
                return c;
            }
            // stream-K: fewer 384-row tiles than CUs, one slice, and every work-group gets at least
            // SCRAPGPU_HIP_MM_SK (default 32) stages. Its partial slots take (CUs + tiles) x 192 KiB
            // of scratch, which the static scratch does not hold (lean). (4096x12288 at 2048 tokens:
            // 213 + 23 (reduce) us against 290 for the 64-token form; at 512 tokens, 16.5 stages per
            // work-group, 69 + 16 against 78: the GEMM is bound by its loads there, 60 KiB per
            // 12.6 MFLOP stage, and the partial sums cost more than the even split saves)
            static const int env_sk = env_int("SCRAPGPU_HIP_MM_SK", 32);
            const int64_t tw = (a.M + 383) / 384 * ntw;
            if (env_sk > 0 && !lean && env_kg != 2 && slices == 1 && stages % 2 == 0 && (a.M % 384 == 0 || a.M >= 8 * 384) && tw < cu_count &&
                tw * stages >= (int64_t) env_sk * cu_count) {
                c.kg = 1;
                c.sk = true;
                return c;
            }
            // ... else K split over work-groups of 384-row tiles when that occupies 2/3 of the CUs
            // or more in one round with >= 16 stages per split (the fewest such splits: the GEMM is
            // bound by its loads there, so more work-groups gain little and every split adds
            // partial sums for k_split_reduce). (4096x12288 at 512 tokens, 44 tiles: 3 / 4 / 5 / 6
            // splits 99 / 88 / 89 / 111 us per op, Q8_0 11008x4096 102 / 92 / 95 / 112, against 95
            // and 92 for the 64-token form's 3 K groups; 6144x4096 at 2 splits on half the CUs
            // lost, 60 against 51)
            if (env_kg != 2 && slices == 1 && (a.M % 384 == 0 || a.M >= 8 * 384))
                for (int sp = 2; sp <= 8; ++sp)
                    if (tw * sp <= cu_count && 3 * tw * sp >= 2 * cu_count && stages / sp >= 16) {
                        c.kg = 1;
                        c.split = sp;
                        return c;
                    }
            c.bn = 64;
            c.wide = false;
        }
        // ... or 384-row x 64-token wave tiles of it (64 tokens or fewer) where they give every CU
        // a work-group at least: the shape is then bound by its
        // weight stream, which the wide form reads from fewer, larger work-groups (the Q6_K LM
        // head at 64 tokens: 163 against 191 us; with fewer tiles than CUs it lost, the 70B-class
        // 28672x8192 at 64 tokens 92 against 77 us split over K)
        if (env_wide != 0 && free_choice && env_kg != 2 && env_kg != 3 && a.K % BK == 0 && a.N <= 64 &&
            (a.M % 384 == 0 || a.M >= 8 * 384) && (a.M + 383) / 384 * ((a.N + 63) / 64) * slices >= cu_count) {
            c.kg = 1;
            c.bn = 64;
            c.wide = true;
            // a second round of tiles at most a quarter full (and >= 16 stages per CU): stream-K
            // over the CUs instead, each an equal run of 2-stage units, the shared tiles added by k_sk_reduce (100000x4096 Q4_K
            // at 64 tokens, 261 tiles: 95.2-96.0 against 109.9-110.1 us; the Q6_K LM head's 396
            // tiles, a second round 55% full, lost: 155 against 140-145)
            const int64_t tw = (a.M + 383) / 384 * ((a.N + 63) / 64);
            static const int env_sk64 = env_int("SCRAPGPU_HIP_MM_SK64", 1);
            if (env_sk64 != 0 && !lean && slices == 1 && stages % 2 == 0 && tw > cu_count && tw < 2 * (int64_t) cu_count &&
                4 * (tw - cu_count) <= cu_count && tw * stages >= 16 * (int64_t) cu_count)
                c.sk = true;
            return c;
        }
        if (env_w == 12) { // forced: KG = 1, split from SCRAPGPU_HIP_MM_SPLIT (the wide GEMM's form where K allows)
            c.kg = 1;
            if (env_split > 0) c.split = (int) std::max<int64_t>(1, std::min<int64_t>(std::min(env_split, 8), (stages + 3) / 4));
            if (env_wide != 0 && a.K % BK == 0) c.wide = true;
            return c;
        }
        if (free_choice) {
            // (each of these tile shapes on the wide GEMM's 64-token form where K is a whole
            // number of stages: 12288x4096 at 128 tokens, K in 4 splits, 36.8-37.0 against
            // 38.7-38.8 us, Q6_K 38.8-38.9 against 40.9)
            if (s12 == 1 && env_kg != 2 && env_kg != 3) {
                c.kg = 1;
                if (env_wide != 0 && a.K % BK == 0) c.wide = true;
                return c;
            }
            if (fits2 && env_kg != 1 && env_kg != 3) {
                // the same 192-row x 64-token tiles on the wide GEMM's 2-K-group form where K is a
                // whole number of stages (x tiles straight into LDS, the exact Q4_K form):
                // 6144x4096 at 512 tokens 46.0-46.5 against 50.9-51.9 us, 12288x4096 at 256 tokens
                // 45.1-45.3 against 50.2
                c.kg = 2;
                if (env_wide != 0 && a.K % BK == 0) c.wide = true;
                return c;
            }
            if (fits3 && env_kg != 1 && env_kg != 2) {
                // (on the wide GEMM's 3-K-group form where K is a whole number of stages: 4096x4096
                // at 512 tokens 38.1-41.3 against 41.4-41.9 us)
                c.kg = 3;
                if (env_wide != 0 && a.K % BK == 0) c.wide = true;
                return c;
            }
            if (s12 > 1 && env_kg != 2 && env_kg != 3) {
                c.kg = 1;
                c.split = s12;
                if (env_wide != 0 && a.K % BK == 0) c.wide = true;
                return c;
            }
        }
    }
    c.w = 4;
    c.kg = 1;
    c.rg = env_rg == 1 || env_rg == 2 ? env_rg : 1;
    const int64_t tm = (a.M + 128 * c.rg - 1) / (128 * c.rg);
    auto tiles = [&](int bn) { return tm * ((a.N + bn - 1) / bn) * slices; };
    // (64 tokens or fewer: BN = 64 and K split to fill the CUs, rather than a half-padding
    // 128-token tile: 38.6 -> 31.0 us on 12288x4096 at N = 64)
    c.bn = env_bn == 64 || env_bn == 128 ? env_bn : (a.N <= 64 || tiles(64) >= occupancy_of(a.dtype, 64, c.rg) * (int64_t) cu_count ? 64 : 128);
    const int64_t want = (int64_t) cu_count * occupancy_of(a.dtype, c.bn, c.rg);
    c.split = 1;
    if (env_split > 0) {
        c.split = (int) std::max<int64_t>(1, std::min<int64_t>(std::min(env_split, 8), (stages + 3) / 4)); // whole groups of 4 stages
        return c;
    }
    while (tiles(c.bn) * c.split < want && stages / (c.split + 1) >= 8 && c.split < 8) ++c.split;
    return c;
}

template <int DT>
void * kernel_of(const MmConfig & c) {
    if (c.sk) return c.bn == 64 ? (void *) k_gemm_w<DT, 1, 2, true> : (void *) k_gemm_w<DT, 1, 4, true>;
    if (c.wide && c.w == 8) return (void *) k_gemm_w<DT, 1, 4, false, false, 8>;
    if (c.wide) return c.bn == 64 ? (c.kg == 3 ? (void *) k_gemm_w<DT, 3, 2> : c.kg == 2 ? (void *) k_gemm_w<DT, 2, 2> : (void *) k_gemm_w<DT, 1, 2>) : c.kg == 2 ? (void *) k_gemm_w<DT, 2> : (void *) k_gemm_w<DT, 1>;
    if (c.w == 12) return c.kg == 3 ? (void *) k_matmul<DT, 64, 1, 12, 3> : c.kg == 2 ? (void *) k_matmul<DT, 64, 1, 12, 2> : (void *) k_matmul<DT, 64, 1, 12, 1>;
    if (c.rg == 1) return c.bn == 64 ? (void *) k_matmul<DT, 64, 1, 4, 1> : (void *) k_matmul<DT, 128, 1, 4, 1>;
    return c.bn == 64 ? (void *) k_matmul<DT, 64, 2, 4, 1> : (void *) k_matmul<DT, 128, 2, 4, 1>;
}

// float weights: the wide GEMM's 12-row-wave form (K split or not), else the 4-wave kernel (their
// raw rows take the registers that its 12-wave and 2-K-group forms need)
template <int DT>
void * kernel_of_float(const MmConfig & c) {
    if (c.wide) return c.kg == 2 ? (void *) k_gemm_w<DT, 2> : (void *) k_gemm_w<DT, 1>;
    return c.bn == 64 ? (void *) k_matmul<DT, 64, 1, 4, 1> : (void *) k_matmul<DT, 128, 1, 4, 1>;
}

// scratch: x as f16 [slices][N][K] | row factors [slices][N] | Q4_K sub-block sums
// [slices][N][xsum_row] | split-K partials
size_t xs_offset(const MatArgs & a) {
    const size_t rows = narrow_shape(a) ? (size_t) (a.N + 31) / 32 * 32 : (size_t) a.N; // (fragment order: whole fragments)
    return (rows * (size_t) a.K * (size_t) (a.ne12 * a.ne13) * sizeof(uint16_t) + 255) / 256 * 256;
}

int64_t xsum_row_of(const MatArgs & a) {
    return a.dtype == Q4_K ? (a.K + 511) / 512 * 16 : 0;
}

size_t xsum_offset(const MatArgs & a) {
    return xs_offset(a) + ((size_t) a.N * (size_t) (a.ne12 * a.ne13) * sizeof(float) + 255) / 256 * 256;
}

size_t part_offset(const MatArgs & a) {
    return xsum_offset(a) + ((size_t) a.N * (size_t) (a.ne12 * a.ne13) * (size_t) xsum_row_of(a) * sizeof(uint16_t) + 255) / 256 * 256;
}

size_t part_bytes(const MatArgs & a, int split) {
    return ((size_t) split * (size_t) (a.ne12 * a.ne13) * (size_t) a.N * (size_t) a.M * sizeof(float) + 255) / 256 * 256;
}

} // namespace

// dynamic LDS beyond the 64 KiB default (gfx950 has 160 KiB per CU): set once per kernel (a
// kernel's LDS size is fixed by its template arguments)
static hipError_t allow_lds(void * fn, size_t lds) {
    if (lds <= 65536) return hipSuccess;
    static std::mutex mu;
    static std::vector<void *> done;
    std::lock_guard<std::mutex> lock(mu);
    if (std::find(done.begin(), done.end(), fn) == done.end()) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
        if (e != hipSuccess) return e;
        done.push_back(fn);
    }
    return hipSuccess;
}

// stream-K partial slots: one per piece, at most cu_count + tiles - 1, each bn x 384 floats. The
// row tiles of 2..3 weights tiled one by one are at most 2 more than those of all their rows
static int64_t sk_max_tiles(const MatArgs & a, int bn) {
    return ((a.M + 383) / 384 + 2) * ((a.N + bn - 1) / bn);
}

static size_t sk_part_bytes(const MatArgs & a, int cu_count, int bn) {
    return (size_t) (cu_count + sk_max_tiles(a, bn) - 1) * bn * 384 * sizeof(float);
}

static bool float_gemm(const MatArgs & a);

template <int DT>
static void * narrow_kernel(int nf, int kw, int rw) {
    if (nf == 1) {
        if (rw == 4) return (void *) k_gemm_n<DT, 1, 4, 4>;
        if (rw == 3) return (void *) k_gemm_n<DT, 1, 4, 3>;
        if (rw == 2) return (void *) k_gemm_n<DT, 1, 8, 2>;
        return kw == 16 ? (void *) k_gemm_n<DT, 1, 16> : (void *) k_gemm_n<DT, 1, 8>;
    }
    if (rw == 2) return (void *) k_gemm_n<DT, 2, 4, 2>;
    if (rw == 3) return (void *) k_gemm_n<DT, 2, 4, 3>;
    return (void *) k_gemm_n<DT, 2, 8>; // (2 fragments in 16 waves would spill: not built)
}

// the narrow GEMM: one work-group per R32 group of each matrix (and slice)
static hipError_t launch_narrow(MmArgs & L, const MatArgs * mats, int nmat, const MmConfig & cfg, hipStream_t stream, const char ** kernel_name) {
    const MatArgs & a = L.a;
    const int nf = cfg.bn / 32 / cfg.nz;
    L.nmat = nmat;
    L.mt[0] = L.mo[0] = 0;
    for (int j = 0; j < 3; ++j) {
        const bool has = j < nmat;
        L.wm[j] = has ? mats[j].w : nullptr;
        L.Mm[j] = has ? mats[j].M : 0;
        L.ym[j] = has ? mats[j].y : nullptr;
        L.ys1m[j] = has ? mats[j].y_s1 : 0;
        L.mt[j + 1] = L.mt[j] + (has ? (mats[j].M + 31) / 32 : 0);
        L.mo[j + 1] = L.mo[j] + (has ? mats[j].M : 0);
    }
    L.tiles_m = L.mt[nmat];
    L.tiles_n = 1;
    L.stages = a.K / BK;
    L.split = 1;
    void * fn = nullptr;
    switch (a.dtype) {
        case Q4_0: fn = narrow_kernel<Q4_0>(nf, cfg.kw, cfg.rw); if (kernel_name) *kernel_name = "matmul_mfma_q4_0"; break;
        case Q8_0: fn = narrow_kernel<Q8_0>(nf, cfg.kw, cfg.rw); if (kernel_name) *kernel_name = "matmul_mfma_q8_0"; break;
        case Q4_K: fn = narrow_kernel<Q4_K>(nf, cfg.kw, cfg.rw); if (kernel_name) *kernel_name = "matmul_mfma_q4_k"; break;
        case Q6_K: fn = narrow_kernel<Q6_K>(nf, cfg.kw, cfg.rw); if (kernel_name) *kernel_name = "matmul_mfma_q6_k"; break;
        default: return hipErrorInvalidValue;
    }
    const size_t lds = (size_t) cfg.rw * (cfg.kw / 2) * nf * 16 * 64 * sizeof(float);
    hipError_t e = allow_lds(fn, lds);
    if (e != hipSuccess) return e;
    const dim3 grid((unsigned) ((L.tiles_m + cfg.rw - 1) / cfg.rw), (unsigned) (a.ne12 * a.ne13), (unsigned) cfg.nz);
    std::snprintf(last_form().form, sizeof(last_form().form), "gemm narrow rw=%d kw=%d bn=%d nz=%d", cfg.rw, cfg.kw, cfg.bn, cfg.nz);
    last_form().grid = (uint64_t) grid.x * grid.y;
    void * args[] = {&L};
    return hipLaunchKernel(fn, grid, dim3((unsigned) (64 * cfg.kw * cfg.rw)), args, lds, stream);
}

size_t matmul_scratch_bytes(const MatArgs & a, int cu_count, bool lean) {
    // (float weights off the GEMM run the float matvec, which takes no scratch)
    if (is_float_weight(a.dtype) && !float_gemm(a)) return 0;
    const MmConfig c = config_of(a, cu_count, lean);
    if (c.sk) return part_offset(a) + sk_part_bytes(a, cu_count, c.bn);
    return part_offset(a) + (c.split == 1 ? 0 : part_bytes(a, c.split));
}

// the pre-pass writes Q4_K's single-fma form of x (high-nibble positions / 16, sub-block sums)
// for the Q4_K kernels that use it, plain scaled x for every other kernel
static bool q4k_x_form(const MatArgs & a, int cu_count, bool lean) {
    const MmConfig c = config_of(a, cu_count, lean);
    return a.dtype == Q4_K && !c.wide && !c.narrow;
}

// x in the narrow GEMM's fragment order
static bool frag_x_form(const MatArgs & a, int cu_count, bool lean) {
    return !is_float_weight(a.dtype) && config_of(a, cu_count, lean).narrow;
}

// float weights on the GEMM: F16 / BF16 with K a whole number of 128-element stages (x rows in bf16
// for BF16); the rest (F32, other K) runs the exact float matvec over groups of 8 columns
static bool float_gemm(const MatArgs & a) {
    return (a.dtype == F16 || a.dtype == BF16) && a.K % BK == 0;
}

bool matmul_reads_same_x(const MatArgs & a, const MatArgs & b) {
    return a.x == b.x && a.x_s1 == b.x_s1 && a.x_s2 == b.x_s2 && a.x_s3 == b.x_s3 && a.N == b.N && a.K == b.K && a.ne12 == b.ne12 &&
           a.ne13 == b.ne13;
}

bool matmul_same_x(const MatArgs & a, const MatArgs & b, int cu_count, bool lean) {
    return matmul_reads_same_x(a, b) && q4k_x_form(a, cu_count, lean) == q4k_x_form(b, cu_count, lean) &&
           frag_x_form(a, cu_count, lean) == frag_x_form(b, cu_count, lean) && (a.dtype == BF16) == (b.dtype == BF16) &&
           !(is_float_weight(a.dtype) && !float_gemm(a)) && !(is_float_weight(b.dtype) && !float_gemm(b));
}

hipError_t launch_matmul_mfma(const MatArgs * mats, int nmat, uint8_t * scratch, int cu_count, hipStream_t stream, const char ** kernel_name,
                              bool x_ready, bool lean) {
    if (nmat < 1 || nmat > 3) return hipErrorInvalidValue;
    // several weights: one slice each, one dtype, the same x; the launch sees them as one matrix
    // of all their rows for its shape choice and scratch
    MatArgs a = mats[0];
    for (int j = 1; j < nmat; ++j) {
        if (mats[j].dtype != a.dtype || !matmul_reads_same_x(mats[j], a) || mats[j].ne12 * mats[j].ne13 != 1 || a.ne12 * a.ne13 != 1) return hipErrorInvalidValue;
        a.M += mats[j].M;
    }
    if (is_float_weight(a.dtype) && !float_gemm(a)) return launch_matvec_float(mats, nmat, stream, kernel_name, nullptr);
    uint16_t * xb = reinterpret_cast<uint16_t *>(scratch);
    const int64_t rows = a.N * a.ne12 * a.ne13;
    float * xs = reinterpret_cast<float *>(scratch + xs_offset(a));
    const bool vec = (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && a.x_s1 % 4 == 0 && a.x_s2 % 4 == 0 && a.x_s3 % 4 == 0;
    uint16_t * xsum = reinterpret_cast<uint16_t *>(scratch + xsum_offset(a));
    const int64_t xsum_row = xsum_row_of(a);
    if (rows > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 xg((unsigned) rows);
    const MmConfig cfg = config_of(a, cu_count, lean);
    if (x_ready) {
        // x converted by the previous product's pre-pass (matmul_same_x)
    } else if (cfg.narrow) {
        if (vec)
            hipLaunchKernelGGL((k_x_to_f16<true, false, false, true>), xg, dim3(256), 0, stream, a, xb, xs, xsum, xsum_row);
        else
            hipLaunchKernelGGL((k_x_to_f16<false, false, false, true>), xg, dim3(256), 0, stream, a, xb, xs, xsum, xsum_row);
    } else if (a.dtype == Q4_K && !cfg.wide) {
        if (vec)
            hipLaunchKernelGGL((k_x_to_f16<true, true>), xg, dim3(256), 0, stream, a, xb, xs, xsum, xsum_row);
        else
            hipLaunchKernelGGL((k_x_to_f16<false, true>), xg, dim3(256), 0, stream, a, xb, xs, xsum, xsum_row);
    } else if (a.dtype == BF16) {
        if (vec)
            hipLaunchKernelGGL((k_x_to_f16<true, false, true>), xg, dim3(256), 0, stream, a, xb, xs, xsum, xsum_row);
        else
            hipLaunchKernelGGL((k_x_to_f16<false, false, true>), xg, dim3(256), 0, stream, a, xb, xs, xsum, xsum_row);
    } else {
        if (vec)
            hipLaunchKernelGGL((k_x_to_f16<true, false>), xg, dim3(256), 0, stream, a, xb, xs, xsum, xsum_row);
        else
            hipLaunchKernelGGL((k_x_to_f16<false, false>), xg, dim3(256), 0, stream, a, xb, xs, xsum, xsum_row);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    MmArgs L;
    std::memset(&L, 0, sizeof(L));
    L.a = a;
    L.xb = xb;
    L.xs = xs;
    L.part = reinterpret_cast<float *>(scratch + part_offset(a));
    if (cfg.narrow) return launch_narrow(L, mats, nmat, cfg, stream, kernel_name);
    L.xsum = xsum;
    L.xsum_row = xsum_row;
    const int BN = cfg.bn;
    const int bmt = 32 * cfg.rg * (cfg.w / cfg.kg);
    // each matrix's rows tiled on their own
    L.nmat = nmat;
    L.mt[0] = L.mo[0] = 0;
    for (int j = 0; j < 3; ++j) {
        const bool has = j < nmat;
        L.wm[j] = has ? mats[j].w : nullptr;
        L.Mm[j] = has ? mats[j].M : 0;
        L.ym[j] = has ? mats[j].y : nullptr;
        L.ys1m[j] = has ? mats[j].y_s1 : 0;
        L.mt[j + 1] = L.mt[j] + (has ? (mats[j].M + bmt - 1) / bmt : 0);
        L.mo[j + 1] = L.mo[j] + (has ? mats[j].M : 0);
    }
    L.packed = 0;
    if (nmat > 1) {
        L.packed = 1;
        for (int j = 0; j + 1 < nmat; ++j)
            if (mats[j].M % (32 * cfg.rg) != 0) L.packed = 0;
    }
    L.tiles_m = L.packed ? (a.M + bmt - 1) / bmt : L.mt[nmat];
    L.tiles_n = (a.N + BN - 1) / BN;
    L.stages = (a.K + BK - 1) / BK;
    L.split = cfg.split;
    // (the wide GEMM with 2 K groups hands half of its sums over through the x buffers at the end)
    size_t lds = cfg.wide ? std::max((size_t) cfg.kg * 2 * BN * XR * sizeof(uint16_t), (size_t) (cfg.kg > 1 ? 12 * 2 * 16 * 64 : 0) * sizeof(float))
                          : (size_t) cfg.kg * 2 * BN * BK * sizeof(uint16_t);
    // (the 8-wave form: one work-group per CU, which more than half of the CU's 160 KiB of LDS
    // ensures; its ~150 VGPRs per lane would also leave room for only one)
    if (cfg.wide && cfg.w == 8) lds = std::max(lds, (size_t) 96 * 1024);
    const int64_t slices = a.ne12 * a.ne13;
    L.sk_g = cfg.sk ? cu_count : 0;
    if (cfg.sk && L.tiles_m * L.tiles_n > sk_max_tiles(a, cfg.bn)) return hipErrorInvalidValue; // (more slots than the scratch holds)
    const dim3 grid(cfg.sk ? (unsigned) cu_count : (unsigned) (L.tiles_m * L.tiles_n * L.split), (unsigned) slices);
    void * args[] = {&L};
    void * fn = nullptr;
    switch (a.dtype) {
        case Q4_0: fn = kernel_of<Q4_0>(cfg); if (kernel_name) *kernel_name = "matmul_mfma_q4_0"; break;
        case Q8_0: fn = kernel_of<Q8_0>(cfg); if (kernel_name) *kernel_name = "matmul_mfma_q8_0"; break;
        case Q4_K: fn = kernel_of<Q4_K>(cfg); if (kernel_name) *kernel_name = "matmul_mfma_q4_k"; break;
        case Q6_K: fn = kernel_of<Q6_K>(cfg); if (kernel_name) *kernel_name = "matmul_mfma_q6_k"; break;
        case F16: fn = kernel_of_float<F16>(cfg); if (kernel_name) *kernel_name = "matmul_mfma_f16"; break;
        case BF16: fn = kernel_of_float<BF16>(cfg); if (kernel_name) *kernel_name = "matmul_mfma_bf16"; break;
        default: return hipErrorInvalidValue;
    }
    if ((e = allow_lds(fn, lds)) != hipSuccess) return e;
    if (cfg.sk)
        std::snprintf(last_form().form, sizeof(last_form().form), "gemm wide stream-k w=12 kg=1 bn=%d rg=1 wgs=%d", BN, cu_count);
    else
        std::snprintf(last_form().form, sizeof(last_form().form), "gemm%s w=%d kg=%d bn=%d rg=%d split=%d", cfg.wide ? " wide" : "", cfg.w, cfg.kg, BN,
                      cfg.rg, L.split);
    last_form().grid = (uint64_t) grid.x * grid.y;
    e = hipLaunchKernel(fn, grid, dim3((unsigned) (64 * cfg.w)), args, lds, stream);
    if (e != hipSuccess || (L.split == 1 && !cfg.sk)) return e;
    bool yvec = a.y_s2 % 4 == 0 && a.y_s3 % 4 == 0;
    for (int j = 0; j < nmat; ++j) yvec = yvec && (reinterpret_cast<uintptr_t>(mats[j].y) & 15) == 0 && mats[j].M % 4 == 0 && mats[j].y_s1 % 4 == 0;
    if (cfg.sk) {
        const dim3 rg((unsigned) (L.tiles_m * L.tiles_n), (unsigned) (BN * 384 / 1024));
        if (BN == 64) {
            if (yvec)
                hipLaunchKernelGGL((k_sk_reduce<true, 64>), rg, dim3(256), 0, stream, L);
            else
                hipLaunchKernelGGL((k_sk_reduce<false, 64>), rg, dim3(256), 0, stream, L);
        } else {
            if (yvec)
                hipLaunchKernelGGL(k_sk_reduce<true>, rg, dim3(256), 0, stream, L);
            else
                hipLaunchKernelGGL(k_sk_reduce<false>, rg, dim3(256), 0, stream, L);
        }
        return hipGetLastError();
    }
    const dim3 rg((unsigned) rows, (unsigned) ((a.M + 1023) / 1024));
    if (yvec)
        hipLaunchKernelGGL(k_split_reduce<true>, rg, dim3(256), 0, stream, L);
    else
        hipLaunchKernelGGL(k_split_reduce<false>, rg, dim3(256), 0, stream, L);
    return hipGetLastError();
}

namespace {

// grouped MUL_MAT_ID: 64-pair tiles once the experts average 16 pairs or more, else 32. An
// expert's last tile is part empty (its MFMAs wasted), but a 32-pair tile feeds each dequantized
// B fragment to one MFMA instead of two: measured (128 experts, 8 used) 32 wins at 8 pairs per
// expert (34 vs 44 us), 64 at 32 (50 vs 56 us)
int ga_bn(const IdArgs & id) {
    static const int env = env_int("SCRAPGPU_HIP_MMID_BN", 0);
    if (env == 32 || env == 64) return env;
    return id.n_used * id.n_tok >= 16 * id.n_exp ? 64 : 32;
}

// the pre-pass's view of MUL_MAT_ID's x: rows t * x_cols + c at x + c * x_s1 + t * x_s2
MatArgs ga_xargs(const MatArgs & a, const IdArgs & id) {
    MatArgs px = a;
    px.N = id.x_shared ? 1 : id.n_used;
    px.ne12 = id.n_tok;
    px.ne13 = 1;
    px.r2 = px.r3 = 1;
    px.x_s3 = 0;
    return px;
}

template <int DT>
void * ga_kernel(int bn, int w) {
    if (w == 12) return bn == 64 ? (void *) k_matmul<DT, 64, 1, 12, 1, true> : (void *) k_matmul<DT, 32, 1, 12, 1, true>;
    return bn == 64 ? (void *) k_matmul<DT, 64, 1, 4, 1, true> : (void *) k_matmul<DT, 32, 1, 4, 1, true>;
}

// grouped MUL_MAT_ID work-groups: 12 waves (384-row tiles, one work-group per CU in step) when
// the experts' row tiles alone (at least one token tile each) come to half the CUs or more
int ga_waves(const MatArgs & a, const IdArgs & id, int cu_count) {
    static const int env = env_int("SCRAPGPU_HIP_MMID_W", 0);
    if (env == 4 || env == 12) return env;
    return id.n_exp * ((a.M + 383) / 384) * 2 >= cu_count ? 12 : 4;
}

} // namespace

size_t mul_mat_id_scratch_bytes(const MatArgs & a, const IdArgs & id) {
    const MatArgs px = ga_xargs(a, id);
    return part_offset(px) + (size_t) (2 * (id.n_exp + 1) + id.n_used * id.n_tok) * sizeof(int32_t);
}

// the grouped path's x form: the wide GEMM (plain f16 x) or k_matmul (its single-fma Q4_K form)
static bool ga_wide(const MatArgs & a, const IdArgs & id, int cu_count) {
    static const int env_wide = env_int("SCRAPGPU_HIP_MM_WIDE", 1);
    return env_wide != 0 && ga_waves(a, id, cu_count) == 12 && ga_bn(id) == 64 && a.K % BK == 0;
}

bool mul_mat_id_same_x(const MatArgs & a, const MatArgs & b, const IdArgs & id, int cu_count) {
    const bool qa = a.dtype == Q4_K && !ga_wide(a, id, cu_count), qb = b.dtype == Q4_K && !ga_wide(b, id, cu_count);
    return a.x == b.x && a.K == b.K && a.x_s1 == b.x_s1 && a.x_s2 == b.x_s2 && qa == qb;
}

hipError_t launch_mul_mat_id_mfma(const MatArgs & a, const IdArgs & id, uint8_t * scratch, int cu_count, hipStream_t stream, const char ** kernel_name,
                                  bool x_ready) {
    const MatArgs px = ga_xargs(a, id);
    const int64_t rows = px.N * id.n_tok;
    if (id.n_exp < 1 || id.n_exp > 1024 || rows * a.K >= ((int64_t) 1 << 31) || id.n_used * id.n_tok >= ((int64_t) 1 << 24)) return hipErrorInvalidValue;
    uint16_t * xb = reinterpret_cast<uint16_t *>(scratch);
    float * xs = reinterpret_cast<float *>(scratch + xs_offset(px));
    uint16_t * xsum = reinterpret_cast<uint16_t *>(scratch + xsum_offset(px));
    const int64_t xsum_row = xsum_row_of(px);
    const bool vec = (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && a.x_s1 % 4 == 0 && a.x_s2 % 4 == 0;
    const int bn = ga_bn(id);
    const int waves = ga_waves(a, id, cu_count);
    // 384-row x 64-token tiles on the wide GEMM where K is a whole number of stages (x tiles
    // straight into LDS, the exact Q4_K form from plain x)
    const bool wide = ga_wide(a, id, cu_count);
    int32_t * e_off = reinterpret_cast<int32_t *>(scratch + part_offset(px));
    int32_t * t_start = e_off + id.n_exp + 1;
    int32_t * pairs = t_start + id.n_exp + 1;
    const RouteArgs ra{id.ids, id.s0, id.s1, (int) id.n_used, (int) id.n_tok, (int) id.n_exp, bn, e_off, t_start, pairs};
    // (work-group 0 routes the pairs, the others convert the x rows)
    const dim3 xrg((unsigned) ((rows + 3) / 4 + 1));
    if (x_ready) {
        // x converted and the pairs routed by the previous grouped MUL_MAT_ID (mul_mat_id_same_x)
    } else if (a.dtype == Q4_K && !wide) {
        if (vec)
            hipLaunchKernelGGL((k_x_route<true, true>), xrg, dim3(1024), 0, stream, px, xb, xs, xsum, xsum_row, rows, ra);
        else
            hipLaunchKernelGGL((k_x_route<false, true>), xrg, dim3(1024), 0, stream, px, xb, xs, xsum, xsum_row, rows, ra);
    } else {
        if (vec)
            hipLaunchKernelGGL((k_x_route<true, false>), xrg, dim3(1024), 0, stream, px, xb, xs, xsum, xsum_row, rows, ra);
        else
            hipLaunchKernelGGL((k_x_route<false, false>), xrg, dim3(1024), 0, stream, px, xb, xs, xsum, xsum_row, rows, ra);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    MmArgs L;
    std::memset(&L, 0, sizeof(L));
    L.a = a;
    L.a.N = bn;
    L.a.ne12 = L.a.ne13 = 1;
    L.xb = xb;
    L.xs = xs;
    L.xsum = xsum;
    L.xsum_row = xsum_row;
    L.part = nullptr;
    L.split = 1;
    L.nmat = 1;
    L.mo[1] = L.mo[2] = L.mo[3] = a.M;
    L.stages = (a.K + BK - 1) / BK;
    L.tiles_m = (a.M + 32 * waves - 1) / (32 * waves);
    L.mt[1] = L.mt[2] = L.mt[3] = L.tiles_m;
    L.tiles_n = (id.n_used * id.n_tok + bn - 1) / bn + id.n_exp; // at least the tiles the routing makes
    L.pairs = pairs;
    L.e_off = e_off;
    L.t_start = t_start;
    L.n_used = (int32_t) id.n_used;
    L.n_exp = (int32_t) id.n_exp;
    L.x_cols = (int32_t) px.N;
    const size_t lds = (size_t) 2 * bn * (wide ? XR : BK) * sizeof(uint16_t) + (size_t) bn * (sizeof(int32_t) + sizeof(int64_t));
    void * fn = nullptr;
    switch (a.dtype) {
        case Q4_0: fn = wide ? (void *) k_gemm_w<Q4_0, 1, 2, false, true> : ga_kernel<Q4_0>(bn, waves); if (kernel_name) *kernel_name = "mul_mat_id_mfma_q4_0"; break;
        case Q8_0: fn = wide ? (void *) k_gemm_w<Q8_0, 1, 2, false, true> : ga_kernel<Q8_0>(bn, waves); if (kernel_name) *kernel_name = "mul_mat_id_mfma_q8_0"; break;
        case Q4_K: fn = wide ? (void *) k_gemm_w<Q4_K, 1, 2, false, true> : ga_kernel<Q4_K>(bn, waves); if (kernel_name) *kernel_name = "mul_mat_id_mfma_q4_k"; break;
        case Q6_K: fn = wide ? (void *) k_gemm_w<Q6_K, 1, 2, false, true> : ga_kernel<Q6_K>(bn, waves); if (kernel_name) *kernel_name = "mul_mat_id_mfma_q6_k"; break;
        default: return hipErrorInvalidValue;
    }
    const int64_t grid = L.tiles_m * L.tiles_n;
    if (grid >= ((int64_t) 1 << 31)) return hipErrorInvalidValue;
    if ((e = allow_lds(fn, lds)) != hipSuccess) return e;
    std::snprintf(last_form().form, sizeof(last_form().form), "grouped%s w=%d bn=%d%s", wide ? " wide" : "", waves, bn, x_ready ? " shared-x" : "");
    last_form().grid = (uint64_t) grid;
    void * args[] = {&L};
    return hipLaunchKernel(fn, dim3((unsigned) grid), dim3((unsigned) (64 * waves)), args, lds, stream);
}

} // namespace sgk
