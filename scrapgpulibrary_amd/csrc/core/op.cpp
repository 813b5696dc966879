// Op descriptor validation and op routing (reference src/core/op.cpp:63-268).
//
// Structural checks apply to every descriptor; the per-op rules are those of the reference's
// contract for the matrix-product family this library executes (MUL_MAT: 2 inputs, 1 output,
// scrapgpu_mul_mat_params present, src0 one of F32/F16/BF16/Q4_0/Q8_0/Q4_K/Q6_K, src1 and dst F32;
// MUL_MAT_MULTI: n weights + the shared x, n outputs, 2 <= n <= 3; MUL_MAT_ID: 3 inputs, 1 output,
// params present). For the remaining op ids only the arity and the parameter block are checked:
// the hip backend reports them UNSUPPORTED with a reason.
#include "scrapgpu/backend.h"

#include <cstddef>
#include <cstring>

namespace {

scrapgpu_status bad(const char * msg) {
    scrapgpu_set_last_error(msg);
    return SCRAPGPU_STATUS_INVALID_ARGUMENT;
}

constexpr size_t kMaxTensors = 32;   // no op takes more than 4 inputs / 2 outputs
constexpr size_t kMaxParams = 4096;  // params are small fixed structs

bool float_weight_or_quant(scrapgpu_dtype t) {
    switch (t) {
        case SCRAPGPU_DTYPE_F32:
        case SCRAPGPU_DTYPE_F16:
        case SCRAPGPU_DTYPE_BF16:
        case SCRAPGPU_DTYPE_Q4_0:
        case SCRAPGPU_DTYPE_Q8_0:
        case SCRAPGPU_DTYPE_Q4_K:
        case SCRAPGPU_DTYPE_Q6_K: return true;
        default: return false;
    }
}

// arity and minimum params size of the ops whose contents this library does not inspect
// (-1: variable arity checked elsewhere)
struct Arity {
    int op, in, out;
    size_t params;
};
const Arity kArity[] = {
    {SCRAPGPU_OP_ADD, 2, 1, 0}, {SCRAPGPU_OP_SUB, 2, 1, 0}, {SCRAPGPU_OP_MUL, 2, 1, 0}, {SCRAPGPU_OP_DIV, 2, 1, 0},
    {SCRAPGPU_OP_SCALE, 1, 1, 2 * sizeof(size_t)}, {SCRAPGPU_OP_CLAMP, 1, 1, 2 * sizeof(size_t)},
    {SCRAPGPU_OP_SQR, 1, 1, 0}, {SCRAPGPU_OP_SQRT, 1, 1, 0}, {SCRAPGPU_OP_RMS_NORM, 1, 1, 0}, {SCRAPGPU_OP_SUM_ROWS, 1, 1, 0},
    {SCRAPGPU_OP_UNARY, 1, 1, 2 * sizeof(size_t)}, {SCRAPGPU_OP_GLU, -1, 1, sizeof(size_t)}, {SCRAPGPU_OP_ROPE, -1, 1, sizeof(size_t)},
    {SCRAPGPU_OP_SOFT_MAX, -1, 1, sizeof(size_t)}, {SCRAPGPU_OP_GET_ROWS, 2, 1, sizeof(size_t)}, {SCRAPGPU_OP_SET_ROWS, 2, 1, sizeof(size_t)},
    {SCRAPGPU_OP_CPY, 1, 1, sizeof(size_t)}, {SCRAPGPU_OP_DUP, 1, 1, 0}, {SCRAPGPU_OP_CONT, 1, 1, 0},
    {SCRAPGPU_OP_ADD_ID, 3, 1, 0}, {SCRAPGPU_OP_SSM_CONV, 2, 1, sizeof(size_t)}, {SCRAPGPU_OP_CONCAT, 2, 1, sizeof(size_t)},
    {SCRAPGPU_OP_PAD, 1, 1, sizeof(size_t)}, {SCRAPGPU_OP_ARGSORT, 1, 1, sizeof(size_t)}, {SCRAPGPU_OP_TOP_K, 1, 1, sizeof(size_t)},
    {SCRAPGPU_OP_RMS_NORM_MUL, 2, 1, sizeof(size_t)}, {SCRAPGPU_OP_ADD_RMS_NORM_MUL, 3, 2, sizeof(size_t)},
    {SCRAPGPU_OP_SET_ROWS_PAIR, 4, 2, 0}, {SCRAPGPU_OP_CONT_MUL_MAT, 2, 1, 0},
};

scrapgpu_status counts(const scrapgpu_op_desc * d, size_t in, size_t out) {
    if (d->input_count != in || d->output_count != out || d->inputs == nullptr || d->outputs == nullptr) {
        return bad("op desc has the wrong input or output count");
    }
    return SCRAPGPU_STATUS_OK;
}

bool params_at_least(const scrapgpu_op_desc * d, size_t n) {
    return d->params != nullptr && d->params_size >= n;
}

} // namespace

extern "C" {

scrapgpu_status scrapgpu_op_desc_validate(const scrapgpu_op_desc * d) {
    if (d == nullptr) return bad("op desc is null");
    if (d->struct_size < offsetof(scrapgpu_op_desc, params_size) + sizeof(d->params_size)) return bad("op desc is null or too small");
    if (d->input_count > kMaxTensors || d->output_count > kMaxTensors) return bad("op desc has an invalid input or output count");
    if ((d->input_count && d->inputs == nullptr) || (d->output_count && d->outputs == nullptr)) return bad("op desc has a null input or output array");
    if (d->params == nullptr && d->params_size > 0) return bad("op desc params_size is set but params is null");
    if (d->params_size > kMaxParams) return bad("op desc params_size is too large");
    for (size_t i = 0; i < d->input_count; ++i)
        if (d->inputs[i].struct_size < sizeof(scrapgpu_tensor_desc)) return bad("input tensor descriptor is too small");
    for (size_t i = 0; i < d->output_count; ++i)
        if (d->outputs[i].struct_size < sizeof(scrapgpu_tensor_desc)) return bad("output tensor descriptor is too small");
    int op_id;
    std::memcpy(&op_id, &d->op, sizeof(op_id));
    switch (op_id) {
        case SCRAPGPU_OP_NONE:
        case SCRAPGPU_OP_RESHAPE:
        case SCRAPGPU_OP_VIEW:
        case SCRAPGPU_OP_PERMUTE:
        case SCRAPGPU_OP_TRANSPOSE: return SCRAPGPU_STATUS_OK;
        case SCRAPGPU_OP_MUL_MAT: {
            if (!params_at_least(d, sizeof(scrapgpu_mul_mat_params))) return bad("MUL_MAT params are missing");
            const scrapgpu_status st = counts(d, 2, 1);
            if (st != SCRAPGPU_STATUS_OK) return st;
            if (!float_weight_or_quant(d->inputs[0].dtype) || d->inputs[1].dtype != SCRAPGPU_DTYPE_F32 ||
                d->outputs[0].dtype != SCRAPGPU_DTYPE_F32) {
                return bad("MUL_MAT dtype contract failed");
            }
            return SCRAPGPU_STATUS_OK;
        }
        case SCRAPGPU_OP_MUL_MAT_MULTI:
            if (d->output_count < 2 || d->output_count > 3 || d->input_count != d->output_count + 1) {
                return bad("MUL_MAT_MULTI takes n+1 inputs and n outputs (2 <= n <= 3)");
            }
            return SCRAPGPU_STATUS_OK;
        case SCRAPGPU_OP_MUL_MAT_ID:
            if (!params_at_least(d, sizeof(scrapgpu_mul_mat_id_params))) return bad("MUL_MAT_ID params are missing");
            return counts(d, 3, 1);
        default: break;
    }
    for (const Arity & a : kArity) {
        if (a.op != op_id) continue;
        if (a.params && !params_at_least(d, a.params)) return bad("op params are missing");
        if (a.in < 0) return counts(d, d->input_count, (size_t) a.out);
        return counts(d, (size_t) a.in, (size_t) a.out);
    }
    return bad("unknown operation");
}

scrapgpu_status scrapgpu_op_supported(scrapgpu_device_t * device, const scrapgpu_op_desc * desc, const char ** reason) {
    scrapgpu_status st = scrapgpu_op_desc_validate(desc);
    if (st == SCRAPGPU_STATUS_OK) {
        const scrapgpu_backend_vtable * vt = device ? reinterpret_cast<const scrapgpu_object_header *>(device)->backend : nullptr;
        if (vt != nullptr && vt->op_supported != nullptr) return vt->op_supported(device, desc, reason);
        scrapgpu_set_last_error("no backend registered for op support query");
        st = SCRAPGPU_STATUS_UNSUPPORTED;
    }
    if (reason != nullptr) *reason = scrapgpu_last_error();
    return st;
}

scrapgpu_status scrapgpu_op_execute(scrapgpu_stream_t * stream, const scrapgpu_op_desc * desc) {
    if (stream == nullptr || desc == nullptr) return bad("stream or op desc is null");
    const scrapgpu_backend_vtable * vt = reinterpret_cast<const scrapgpu_object_header *>(stream)->backend;
    if (vt == nullptr) return bad("stream does not belong to a registered backend");
    if (vt->op_execute == nullptr) {
        scrapgpu_set_last_error("the stream backend cannot execute ops");
        return SCRAPGPU_STATUS_UNSUPPORTED;
    }
    return vt->op_execute(stream, desc);
}

}
