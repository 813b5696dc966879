// Exposes the reference's own R32 host pack/unpack (src/backends/opencl11/r32.h:35-90, inline in
// that header) and R32 geometry (src/tensor/tensor.cpp) as C symbols of oracle/_ref, so that tests
// can compare the oracle's R32 restatement with the reference code compiled from source. Only the
// reference's functions run; this file holds the C entry points and the per-slice area addressing
// of the reference's r32 tests (tests/r32/r32_tests.cpp:33-57).
#include "opencl11/r32.h"

extern "C" int ref_r32_move(int dtype, int64_t K, int64_t M, int64_t slices, uint8_t * nat, uint8_t * rep, int pack) {
    const int64_t ne[4] = {K, M, slices, 1};
    const sgt::TensorDesc d = sgt::make_contiguous((scrapgpu_dtype) dtype, ne);
    if (!sgt::r32_eligible(d)) return 1;
    const sgt::r32_geom g = sgt::r32_geometry(d);
    const size_t slice = (size_t) g.M * g.rowb;
    for (int64_t s = 0; s < slices; ++s) {
        uint8_t * ap[3] = {nullptr, nullptr, nullptr};
        for (int k = 0; k < g.na; ++k) {
            ap[k] = rep + (size_t) s * slice + (size_t) g.M * (size_t) g.nb * sgt::r32_area_before(g, k);
        }
        if (pack) {
            cl11_rp_pack(g, nat + (size_t) s * slice, g.M, ap);
        } else {
            cl11_rp_unpack(g, (const uint8_t * const *) ap, g.M, nat + (size_t) s * slice);
        }
    }
    return 0;
}
