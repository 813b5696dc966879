// Tensor descriptor math shared by the core and the hip backend: dtype sizes, contiguity, the R32
// eligibility rule and the R32 geometry. Restates the semantics of the reference's
// src/tensor/tensor.h:26-76,180-250,343-398 and src/tensor/tensor.cpp:5-19.
#pragma once

#include "scrapgpu/tensor.h"

#include <cstddef>
#include <cstdint>
#include <limits>

namespace sg {

inline size_t type_size(scrapgpu_dtype t) {
    switch (t) {
        case SCRAPGPU_DTYPE_F32: return 4;
        case SCRAPGPU_DTYPE_F16: return 2;
        case SCRAPGPU_DTYPE_I32: return 4;
        case SCRAPGPU_DTYPE_I64: return 8;
        case SCRAPGPU_DTYPE_I16: return 2;
        case SCRAPGPU_DTYPE_BF16: return 2;
        case SCRAPGPU_DTYPE_Q4_0: return 18;
        case SCRAPGPU_DTYPE_Q8_0: return 34;
        case SCRAPGPU_DTYPE_Q4_K: return 144;
        case SCRAPGPU_DTYPE_Q6_K: return 210;
        default: return 0;
    }
}

inline size_t block_size(scrapgpu_dtype t) {
    switch (t) {
        case SCRAPGPU_DTYPE_Q4_0:
        case SCRAPGPU_DTYPE_Q8_0: return 32;
        case SCRAPGPU_DTYPE_Q4_K:
        case SCRAPGPU_DTYPE_Q6_K: return 256;
        default: return type_size(t) != 0 ? 1 : 0;
    }
}

inline bool is_quant(scrapgpu_dtype t) {
    return t == SCRAPGPU_DTYPE_Q4_0 || t == SCRAPGPU_DTYPE_Q8_0 || t == SCRAPGPU_DTYPE_Q4_K || t == SCRAPGPU_DTYPE_Q6_K;
}

inline int64_t dim1(int64_t ne) {
    return ne <= 0 ? 1 : ne;
}

inline size_t row_size(scrapgpu_dtype t, int64_t ne0) {
    const size_t bs = block_size(t), ts = type_size(t);
    if (ne0 < 0 || bs == 0) return 0;
    const uint64_t blocks = ((uint64_t) ne0 + bs - 1) / bs;
    if (blocks > std::numeric_limits<size_t>::max() / ts) return 0;
    return (size_t) blocks * ts;
}

inline uint64_t sat_mul(uint64_t a, uint64_t b) {
    return a != 0 && b > std::numeric_limits<uint64_t>::max() / a ? std::numeric_limits<uint64_t>::max() : a * b;
}

inline uint64_t sat_add(uint64_t a, uint64_t b) {
    return b > std::numeric_limits<uint64_t>::max() - a ? std::numeric_limits<uint64_t>::max() : a + b;
}

// bytes spanned by the tensor from its first element (ggml's nbytes; 0 if a dim is <= 0)
inline uint64_t nbytes(const scrapgpu_tensor_desc & d) {
    for (int i = 0; i < 4; ++i)
        if (d.ne[i] <= 0) return 0;
    const size_t bs = block_size(d.dtype), ts = type_size(d.dtype);
    if (bs == 0) return 0;
    uint64_t n = bs == 1 ? ts : sat_mul((uint64_t) d.ne[0], d.nb[0]) / bs;
    for (int i = bs == 1 ? 0 : 1; i < 4; ++i) n = sat_add(n, sat_mul((uint64_t) (d.ne[i] - 1), d.nb[i]));
    return n;
}

// ggml contiguity: dims of size 1 (and nb0 of a one-block row) are unconstrained
inline bool contiguous_ggml(const scrapgpu_tensor_desc & d) {
    const size_t bs = block_size(d.dtype);
    uint64_t expect = type_size(d.dtype);
    if (bs == 0 || expect == 0) return false;
    if (d.ne[0] != (int64_t) bs && d.nb[0] != expect) return false;
    bool overflow = (uint64_t) (d.ne[0] / (int64_t) bs) > std::numeric_limits<uint64_t>::max() / expect;
    expect *= (uint64_t) (d.ne[0] / (int64_t) bs);
    for (int i = 1; i < 4; ++i) {
        if (d.ne[i] != 1 && d.nb[i] != expect) return false;
        overflow |= expect != 0 && (uint64_t) d.ne[i] > std::numeric_limits<uint64_t>::max() / expect;
        expect *= (uint64_t) d.ne[i];
    }
    return !overflow;
}

// every stride is exactly the canonical one (the public scrapgpu_tensor_is_contiguous)
inline bool contiguous_strict(const scrapgpu_tensor_desc & d) {
    const size_t row = row_size(d.dtype, dim1(d.ne[0]));
    if (row == 0 || d.nb[0] != type_size(d.dtype)) return false;
    uint64_t expect = row;
    for (int i = 1; i < 4; ++i) {
        if (d.nb[i] != expect) return false;
        const uint64_t n = (uint64_t) dim1(d.ne[i]);
        if (expect > std::numeric_limits<uint64_t>::max() / n) return false;
        expect *= n;
    }
    return true;
}

inline bool r32_eligible(const scrapgpu_tensor_desc & d) {
    if (!is_quant(d.dtype) || !contiguous_ggml(d)) return false;
    if (d.ne[0] <= 0 || (uint64_t) d.ne[0] % block_size(d.dtype) != 0) return false;
    return (d.ne[2] == 1 && d.ne[3] == 1) || (d.nb[2] % 16 == 0 && d.nb[3] % 16 == 0);
}

// R32: the bytes of a natural block are split into up to 3 areas laid out one after the other in
// each slice (area k starts at M * nb * sum of the earlier areas' bytes per block). Rows are grouped
// by 32 (rs = rows of the group, fewer in the last group of a slice). Inside an area of 16*U bytes
// per block, group g starts at g * 32 * nb * 16U and 16-byte unit j of block b of row `lane` is unit
// (b*U + j) * rs + lane of the group; an area of 2 bytes holds halves at b * rs + lane.
struct R32Area {
    int src;      // first byte of the area inside the natural block
    int len;      // bytes per block (2, or a multiple of 16)
    uint8_t xr;   // xor mask applied to the bytes
};

struct R32Geom {
    int na = 0;
    R32Area area[3] = {};
    int64_t M = 0;   // rows per slice
    int64_t nb = 0;  // blocks per row
    int bs = 0;      // bytes per natural block
    size_t rowb = 0; // bytes per natural row
    uint64_t area_off(int k) const {
        uint64_t before = 0;
        for (int i = 0; i < k; ++i) before += (uint64_t) area[i].len;
        return (uint64_t) M * (uint64_t) nb * before;
    }
};

inline R32Geom r32_geometry(scrapgpu_dtype t, int64_t K, int64_t M) {
    R32Geom g;
    g.M = M;
    g.bs = (int) type_size(t);
    g.nb = block_size(t) ? K / (int64_t) block_size(t) : 0;
    g.rowb = (size_t) g.nb * (size_t) g.bs;
    switch (t) {
        case SCRAPGPU_DTYPE_Q8_0: g.na = 2; g.area[0] = {2, 32, 0x80}; g.area[1] = {0, 2, 0}; break;
        case SCRAPGPU_DTYPE_Q4_0: g.na = 2; g.area[0] = {2, 16, 0}; g.area[1] = {0, 2, 0}; break;
        case SCRAPGPU_DTYPE_Q4_K: g.na = 2; g.area[0] = {16, 128, 0}; g.area[1] = {0, 16, 0}; break;
        case SCRAPGPU_DTYPE_Q6_K: g.na = 3; g.area[0] = {0, 192, 0}; g.area[1] = {192, 16, 0x80}; g.area[2] = {208, 2, 0}; break;
        default: break;
    }
    return g;
}

} // namespace sg
