/* Tensor descriptors (reference include/scrapgpu/tensor.h:10-73).
 *
 * ggml orientation: ne[0] is the contiguous (inner) dim, nb[] are byte strides, a quantized dtype
 * is stored in blocks of scrapgpu_dtype_block_size() elements. `layout` is the physical layout of
 * the whole tensor: SCRAPGPU_LAYOUT_R32 stores a Q4_0/Q8_0/Q4_K/Q6_K tensor regrouped by 32 rows
 * (the byte arrangement is described in scrapgpulibrary_amd/csrc/core/r32.h); its device bytes
 * have the same size as the natural bytes, and host transfers always carry the natural layout. */
#ifndef SCRAPGPU_TENSOR_H
#define SCRAPGPU_TENSOR_H

#include "scrapgpu/buffer.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum scrapgpu_dtype {
    SCRAPGPU_DTYPE_UNKNOWN = -1,
    SCRAPGPU_DTYPE_F32 = 0,
    SCRAPGPU_DTYPE_F16 = 1,
    SCRAPGPU_DTYPE_I32 = 2,
    SCRAPGPU_DTYPE_I64 = 3,
    SCRAPGPU_DTYPE_I16 = 4,
    SCRAPGPU_DTYPE_BF16 = 5,
    SCRAPGPU_DTYPE_Q4_0 = 16,
    SCRAPGPU_DTYPE_Q8_0 = 17,
    SCRAPGPU_DTYPE_Q4_K = 32,
    SCRAPGPU_DTYPE_Q6_K = 33,
} scrapgpu_dtype;

typedef enum scrapgpu_layout {
    SCRAPGPU_LAYOUT_NATURAL = 0,
    SCRAPGPU_LAYOUT_R32 = 1,
} scrapgpu_layout;

typedef struct scrapgpu_tensor_desc {
    size_t struct_size;
    scrapgpu_dtype dtype;
    int64_t ne[4];
    uint64_t nb[4];
    scrapgpu_buffer_t * buffer;
    uint64_t offset;
    scrapgpu_layout layout;
} scrapgpu_tensor_desc;

SCRAPGPU_API size_t scrapgpu_dtype_block_size(scrapgpu_dtype dtype);
SCRAPGPU_API size_t scrapgpu_dtype_type_size(scrapgpu_dtype dtype);
SCRAPGPU_API size_t scrapgpu_tensor_row_size(scrapgpu_dtype dtype, int64_t ne0);
SCRAPGPU_API int scrapgpu_tensor_is_contiguous(const scrapgpu_tensor_desc * desc);
SCRAPGPU_API int scrapgpu_tensor_r32_eligible(const scrapgpu_tensor_desc * desc);

/* Host <-> device transfer of the first `size` natural-layout bytes of the tensor (reference
 * tensor.h:45-52, registry.cpp:186-198). An R32 tensor is packed / unpacked on the way (on the
 * device, in HBM). The call is synchronous with respect to the host pointer. */
SCRAPGPU_API scrapgpu_status scrapgpu_tensor_upload(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * desc, const void * host, size_t size);
SCRAPGPU_API scrapgpu_status scrapgpu_tensor_download(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * desc, void * host, size_t size);

#ifdef __cplusplus
}
#endif

#endif
