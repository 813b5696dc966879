// Op descriptor validation and op routing (reference src/core/op.cpp:63-268).
//
// Structural checks apply to every descriptor; the per-op rules are those of the reference's
// contract for the matrix-product family this library executes (MUL_MAT: 2 inputs, 1 output,
// scrapgpu_mul_mat_params present, src0 one of F32/F16/BF16/Q4_0/Q8_0/Q4_K/Q6_K, src1 and dst F32;
// MUL_MAT_MULTI: n weights + the shared x, n outputs, 2 <= n <= 3; MUL_MAT_ID: 3 inputs, 1 output,
// params present). For the remaining op ids only the arity and the parameter block are checked:
// the hip backend reports them UNSUPPORTED with a reason.
#include "dispatch.h"

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
        return bad("this op takes a different number of inputs or outputs");
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
    if (d->struct_size < offsetof(scrapgpu_op_desc, params_size) + sizeof(d->params_size)) return bad("the op desc is null or shorter than its required fields");
    if (d->input_count > kMaxTensors || d->output_count > kMaxTensors) return bad("the op desc's input or output count is out of range");
    if ((d->input_count && d->inputs == nullptr) || (d->output_count && d->outputs == nullptr)) return bad("the op desc lists tensors but its input or output array is null");
    if (d->params == nullptr && d->params_size > 0) return bad("the op desc has a params_size but no params");
    if (d->params_size > kMaxParams) return bad("the op desc's params_size is implausibly large");
    for (size_t i = 0; i < d->input_count; ++i)
        if (d->inputs[i].struct_size < sizeof(scrapgpu_tensor_desc)) return bad("an input tensor desc is shorter than its required fields");
    for (size_t i = 0; i < d->output_count; ++i)
        if (d->outputs[i].struct_size < sizeof(scrapgpu_tensor_desc)) return bad("an output tensor desc is shorter than its required fields");
    int op_id;
    std::memcpy(&op_id, &d->op, sizeof(op_id));
    switch (op_id) {
        case SCRAPGPU_OP_NONE:
        case SCRAPGPU_OP_RESHAPE:
        case SCRAPGPU_OP_VIEW:
        case SCRAPGPU_OP_PERMUTE:
        case SCRAPGPU_OP_TRANSPOSE: return SCRAPGPU_STATUS_OK;
        case SCRAPGPU_OP_MUL_MAT: {
            if (!params_at_least(d, sizeof(scrapgpu_mul_mat_params))) return bad("MUL_MAT needs its params (scrapgpu_mul_mat_params)");
            const scrapgpu_status st = counts(d, 2, 1);
            if (st != SCRAPGPU_STATUS_OK) return st;
            if (!float_weight_or_quant(d->inputs[0].dtype) || d->inputs[1].dtype != SCRAPGPU_DTYPE_F32 ||
                d->outputs[0].dtype != SCRAPGPU_DTYPE_F32) {
                return bad("MUL_MAT: src0 must be F32/F16/BF16/Q4_0/Q8_0/Q4_K/Q6_K and src1, dst F32");
            }
            return SCRAPGPU_STATUS_OK;
        }
        case SCRAPGPU_OP_MUL_MAT_MULTI:
            if (d->output_count < 2 || d->output_count > 3 || d->input_count != d->output_count + 1) {
                return bad("MUL_MAT_MULTI: 2 or 3 weights, then the shared src1, and one output per weight");
            }
            return SCRAPGPU_STATUS_OK;
        case SCRAPGPU_OP_MUL_MAT_ID:
            if (!params_at_least(d, sizeof(scrapgpu_mul_mat_id_params))) return bad("MUL_MAT_ID needs its params (scrapgpu_mul_mat_id_params)");
            return counts(d, 3, 1);
        default: break;
    }
    for (const Arity & a : kArity) {
        if (a.op != op_id) continue;
        if (a.params && !params_at_least(d, a.params)) return bad("op params are missing");
        if (a.in < 0) return counts(d, d->input_count, (size_t) a.out);
        return counts(d, (size_t) a.in, (size_t) a.out);
    }
    return bad("the op id is not one this API defines");
}

scrapgpu_status scrapgpu_op_supported(scrapgpu_device_t * device, const scrapgpu_op_desc * desc, const char ** reason) {
    const char * call = "scrapgpu_op_supported";
    scrapgpu_status st = scrapgpu_op_desc_validate(desc);
    if (st == SCRAPGPU_STATUS_OK) {
        const scrapgpu_backend_vtable * t = sgcore::owner_table(device, call, "device");
        if (t == nullptr) {
            st = SCRAPGPU_STATUS_UNSUPPORTED; // (no backend to ask: the op is not supported here)
        } else if (t->op_supported == nullptr) {
            st = sgcore::not_implemented(call, t, "op_supported");
        } else {
            return t->op_supported(device, desc, reason);
        }
    }
    if (reason != nullptr) *reason = scrapgpu_last_error();
    return st;
}

scrapgpu_status scrapgpu_op_execute(scrapgpu_stream_t * stream, const scrapgpu_op_desc * desc) {
    const char * call = "scrapgpu_op_execute";
    if (desc == nullptr) return sgcore::null_argument(call, "desc");
    const scrapgpu_backend_vtable * t = sgcore::owner_table(stream, call, "stream");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->op_execute == nullptr) return sgcore::not_implemented(call, t, "op_execute");
    return t->op_execute(stream, desc);
}

}
