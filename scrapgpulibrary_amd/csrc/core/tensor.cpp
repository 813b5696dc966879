// Public tensor helpers (reference src/core/tensor.cpp:1-35 over src/tensor/tensor.h).
#include "scrapgpu/tensor.h"

#include "tensor_math.h"

extern "C" {

size_t scrapgpu_dtype_block_size(scrapgpu_dtype dtype) {
    return sg::block_size(dtype);
}

size_t scrapgpu_dtype_type_size(scrapgpu_dtype dtype) {
    return sg::type_size(dtype);
}

size_t scrapgpu_tensor_row_size(scrapgpu_dtype dtype, int64_t ne0) {
    return sg::row_size(dtype, ne0);
}

int scrapgpu_tensor_is_contiguous(const scrapgpu_tensor_desc * desc) {
    return desc != nullptr && sg::contiguous_strict(*desc) ? 1 : 0;
}

int scrapgpu_tensor_r32_eligible(const scrapgpu_tensor_desc * desc) {
    return desc != nullptr && sg::r32_eligible(*desc) ? 1 : 0;
}

}
