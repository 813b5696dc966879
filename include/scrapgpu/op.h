/* Op descriptors (reference include/scrapgpu/op.h:10-48, 165-200).
 *
 * The op enum is ABI and lists every op id of the reference. This library implements the
 * quantized matrix-product family (MUL_MAT, MUL_MAT_MULTI) on the hip backend; every other op is
 * answered with SCRAPGPU_STATUS_UNSUPPORTED and a reason by op_supported / op_execute. Only the
 * parameter structs of the ops this library reads are declared here. */
#ifndef SCRAPGPU_OP_H
#define SCRAPGPU_OP_H

#include "scrapgpu/tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum scrapgpu_op {
    SCRAPGPU_OP_NONE = 0,
    SCRAPGPU_OP_RESHAPE = 1,
    SCRAPGPU_OP_VIEW = 2,
    SCRAPGPU_OP_PERMUTE = 3,
    SCRAPGPU_OP_TRANSPOSE = 4,
    SCRAPGPU_OP_ADD = 10,
    SCRAPGPU_OP_SUB = 11,
    SCRAPGPU_OP_MUL = 12,
    SCRAPGPU_OP_DIV = 13,
    SCRAPGPU_OP_SCALE = 14,
    SCRAPGPU_OP_CLAMP = 15,
    SCRAPGPU_OP_SQR = 16,
    SCRAPGPU_OP_SQRT = 17,
    SCRAPGPU_OP_UNARY = 18,
    SCRAPGPU_OP_GLU = 19,
    SCRAPGPU_OP_RMS_NORM = 20,
    SCRAPGPU_OP_ROPE = 21,
    SCRAPGPU_OP_SOFT_MAX = 22,
    SCRAPGPU_OP_GET_ROWS = 23,
    SCRAPGPU_OP_SET_ROWS = 24,
    SCRAPGPU_OP_CPY = 25,
    SCRAPGPU_OP_DUP = 26,
    SCRAPGPU_OP_CONT = 27,
    SCRAPGPU_OP_MUL_MAT = 28,
    SCRAPGPU_OP_MUL_MAT_ID = 29,
    SCRAPGPU_OP_ADD_ID = 30,
    SCRAPGPU_OP_SSM_CONV = 31,
    SCRAPGPU_OP_CONCAT = 32,
    SCRAPGPU_OP_PAD = 33,
    SCRAPGPU_OP_SUM_ROWS = 34,
    SCRAPGPU_OP_ARGSORT = 35,
    SCRAPGPU_OP_TOP_K = 36,
    SCRAPGPU_OP_RMS_NORM_MUL = 100,
    SCRAPGPU_OP_ADD_RMS_NORM_MUL = 101,
    SCRAPGPU_OP_SET_ROWS_PAIR = 102,
    SCRAPGPU_OP_MUL_MAT_MULTI = 103,
    SCRAPGPU_OP_CONT_MUL_MAT = 104,
} scrapgpu_op;

/* GET_ROWS (reference op.h:145-148): inputs [src0 (K x R per slice), ids (I32)], output
 * [dst F32 (K x ids)]: dst[:, a, b, c] = row ids[a, b, c] of slice (b, c), dequantized. The hip
 * backend reads R32 rows; indices outside [0, R) read the nearest row. */
typedef struct scrapgpu_get_rows_params {
    size_t struct_size;
    int indices_are_i64;
} scrapgpu_get_rows_params;

/* MUL_MAT: inputs [src0 = W (K x M per slice), src1 = x (K x N)], output [dst (M x N)].
 * allow_broadcast != 0 lets src1 dims 2/3 be multiples of src0's (reference op.h:165-168). */
typedef struct scrapgpu_mul_mat_params {
    size_t struct_size;
    int allow_broadcast;
} scrapgpu_mul_mat_params;

/* MUL_MAT_ID (reference op.h:170-174): inputs [src0 = experts (K x M x E), src1 = x (K x 1|n_used
 * x n_tokens), ids (I32 n_used x n_tokens)], output [dst (M x n_used x n_tokens)]. The hip backend
 * reads the ids on the device (indices outside [0, E) are clamped, like the reference's GPU
 * kernels); n_used and max_prompt_tokens are not needed by it. */
typedef struct scrapgpu_mul_mat_id_params {
    size_t struct_size;
    uint32_t n_used;
    uint32_t max_prompt_tokens;
} scrapgpu_mul_mat_id_params;

typedef struct scrapgpu_op_desc {
    size_t struct_size;
    scrapgpu_op op;
    const scrapgpu_tensor_desc * inputs;
    size_t input_count;
    scrapgpu_tensor_desc * outputs;
    size_t output_count;
    const void * params;
    size_t params_size;
} scrapgpu_op_desc;

SCRAPGPU_API scrapgpu_status scrapgpu_op_desc_validate(const scrapgpu_op_desc * desc);
SCRAPGPU_API scrapgpu_status scrapgpu_op_supported(scrapgpu_device_t * device, const scrapgpu_op_desc * desc, const char ** reason);

/* Executes one op on the stream's device (a one-node plan); asynchronous, results visible after
 * scrapgpu_stream_sync or a blocking read (reference op.h:186-194). */
SCRAPGPU_API scrapgpu_status scrapgpu_op_execute(scrapgpu_stream_t * stream, const scrapgpu_op_desc * desc);

#ifdef __cplusplus
}
#endif

#endif
