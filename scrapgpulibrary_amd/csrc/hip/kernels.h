// Launch interface between the hip backend's host code and its gfx950 kernels. Plain pointers,
// sizes and strides only; every function enqueues on `stream` and returns the launch error.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sgk {

enum : int { F32 = 0, F16 = 1, BF16 = 5, Q4_0 = 16, Q8_0 = 17, Q4_K = 32, Q6_K = 33 };

// The form the calling thread's last matvec / matmul launch chose ("burst rg=3 W=4 spw=2", ...)
// and its work-group count: a diagnostic that lets tests pin the kernel a shape selects.
struct LaunchForm {
    char form[96];
    uint64_t grid;
};
LaunchForm & last_form();

// R32 area table of one dtype (the same numbers as sg::r32_geometry)
struct Areas {
    int na;
    int src[3];
    int len[3];
    uint8_t xr[3];
};
Areas areas_of(int dtype);

// Matrix product y[n, m] = sum_k W[m, k] x[n, k] over R32 quantized weights or natural-layout
// float weights (F32 / F16 / BF16). W: slices of M rows, nb blocks each (quantized) or rows nb
// bytes apart (float); slice (i2/r2, i3/r3) starts at w + i2w * w_s2 + i3w * w_s3 (bytes). x / y:
// float element strides (s1 between columns, s2 / s3 between slices).
struct MatArgs {
    int dtype;
    const uint8_t * w;
    uint64_t w_s2, w_s3;
    int64_t M, K, nb;
    const float * x;
    int64_t x_s1, x_s2, x_s3;
    float * y;
    int64_t y_s1, y_s2, y_s3;
    int64_t N;          // columns of x / y
    int64_t ne12, ne13; // dst slices
    int64_t r2, r3;     // broadcast factors
};

// MUL_MAT_ID: the slices of a matvec are the (slot i, token t) pairs, pair = t * n_used + i; the
// expert e = ids[i * s0 + t * s1] (I32, read on the device, clamped to [0, n_exp)) selects the
// weights at w + e * w_s2; x column (x_shared ? 0 : i) of token t (x + i * x_s1 + t * x_s2);
// y column i of token t (y + i * y_s1 + t * y_s2).
struct IdArgs {
    const int32_t * ids;
    int64_t s0, s1;       // element strides of ids
    int64_t n_used, n_tok, n_exp;
    int x_shared;         // src1 has one column per token, shared by the slots
};

// decode matvec for 1 <= N <= 8 (weights streamed once, every column reused in registers).
// nmat = 1, or 2..3 single-slice products of one dtype and K that share x (one fused launch;
// mats[j].w / M / y / y_s1 per matrix, everything else from mats[0]). With `id` (N = 1): the
// MUL_MAT_ID pairs above instead of the slices; nmat > 1 expert tensors then share the ids, x, the
// expert stride w_s2 and the output strides y_s1 / y_s2.
// Scratch the launch needs: for 2..8 columns of one slice, x converted once to its int8 planes,
// and the partial sums of K chunks when K > 4096. launch_matvec takes that much device memory as
// `scratch` (null: the form that needs none).
// One column with a long K (17..64 steps of 256) on one slice: K in chunks of 16 steps over
// separate work-groups, whose partial sums take matvec_scratch_bytes of `scratch` and meet through
// `arrive`: kArriveMax counters that must be zero before the first launch that uses them and are
// left at zero by every launch (the last chunk of a row tile resets its count); launches that
// share them must not overlap. Without scratch or counters the one-work-group-per-tile form runs.
constexpr int64_t kArriveMax = 65536;
bool is_float_weight(int dtype);
// float weights (launch_matvec calls it for them, launch_matmul_mfma for F32 and for K not a
// multiple of 128): exact f32 products, K a multiple of 8, rows and slices 16-byte aligned; one
// launch per group of 8 columns; no scratch
// With `id` (N = 1): the MUL_MAT_ID pairs as launch_matvec takes them.
hipError_t launch_matvec_float(const MatArgs * mats, int nmat, hipStream_t stream, const char ** kernel_name, uint64_t * grid_size,
                               const IdArgs * id = nullptr);
size_t matvec_scratch_bytes(const MatArgs * mats, int nmat, const IdArgs * id = nullptr);
hipError_t launch_matvec(const MatArgs * mats, int nmat, int cu_count, hipStream_t stream, const char ** kernel_name,
                         uint64_t * grid_size, const IdArgs * id = nullptr, uint8_t * scratch = nullptr, uint32_t * arrive = nullptr);

// prefill: f16 MFMA with fp32 accumulate, weights dequantized in registers (any N >= 1).
// `scratch` (matmul_scratch_bytes(a, cu_count) bytes of device memory, owned by the stream)
// receives x as scaled f16 rows with their factors and, when K is split over work-groups, the
// partial sums.
// nmat = 1, or 2..3 single-slice weights of one dtype that read the same x (matmul_reads_same_x): one
// launch over all their row tiles (run end to end over all their rows when every weight but the
// last has a whole number of a wave's 32 or 64 rows); matmul_scratch_bytes then takes mats[0] with M = the sum of the
// matrices' M. `lean`: only forms whose scratch is the x buffers and at most split-K partials (no
// stream-K slots), for a caller whose scratch is a fixed static array; the same `lean` must be
// passed to every call about one launch.
size_t matmul_scratch_bytes(const MatArgs & a, int cu_count, bool lean = false);
hipError_t launch_matmul_mfma(const MatArgs * mats, int nmat, uint8_t * scratch, int cu_count, hipStream_t stream, const char ** kernel_name,
                              bool x_ready = false, bool lean = false);
// true when b's x pre-pass would write what a's did (same x and shape, and the same x form: the
// Q4_K single-fma kernels read x in a form of their own): a product
// launched right after a's on the same scratch may then pass x_ready and skip its own
bool matmul_same_x(const MatArgs & a, const MatArgs & b, int cu_count, bool lean = false);
// true when a and b read the same x with the same shape (what one fused launch over both needs)
bool matmul_reads_same_x(const MatArgs & a, const MatArgs & b);

// MUL_MAT_ID with many tokens (prefill): the (slot, token) pairs are grouped by expert on the
// device (ids clamped as above), x goes through the matmul's pre-pass once, and the f16 MFMA GEMM
// runs over (expert, 32- or 64-pair tile, 128- or 384-row tile) with gathered x rows and scattered
// outputs; each expert's weights are read once per row tile instead of once per pair. `scratch`:
// mul_mat_id_scratch_bytes(a, id) bytes (a as mul_mat_id_rule fills it; a.N = 1).
// x_ready: the scratch already holds this x's pre-pass output and these ids' routing (the
// previous launch on it was a grouped MUL_MAT_ID for which mul_mat_id_same_x(prev, a, id) held),
// so only the GEMM is launched.
size_t mul_mat_id_scratch_bytes(const MatArgs & a, const IdArgs & id);
hipError_t launch_mul_mat_id_mfma(const MatArgs & a, const IdArgs & id, uint8_t * scratch, int cu_count, hipStream_t stream,
                                  const char ** kernel_name, bool x_ready = false);
// true when grouped MUL_MAT_IDs a and b over the same x and ids (one IdArgs) write the same
// pre-pass output and routing: the same x form and token tile, so b may run with x_ready after a
bool mul_mat_id_same_x(const MatArgs & a, const MatArgs & b, const IdArgs & id, int cu_count);

// GET_ROWS on R32 weights: dst[:, a, b, c] = dequantized row ids[a, b, c] of slice (b, c) of src0
// (bit-exact with the dequantizer; out-of-range indices read the nearest row).
struct GetRowsLaunch {
    int dtype;            // quantized (R32) or F32 / F16 (natural rows w_s1 bytes apart)
    const uint8_t * w;
    uint64_t w_s1, w_s2, w_s3;
    const int32_t * ids;
    int64_t i_s0, i_s1, i_s2; // element strides
    float * y;
    int64_t y_s1, y_s2, y_s3; // element strides
    int64_t K, M, n0, n1, n2; // src0 ne0, ne1; ids ne0..2
};
hipError_t launch_get_rows(const GetRowsLaunch & g, hipStream_t stream);

// R32 pack (natural -> R32) or unpack of rows [row0, row0 + nrows) of one slice of M rows; row0 is
// a multiple of 32. `nat` holds the natural bytes of those rows, `rep` is the slice's R32 base.
hipError_t launch_r32_move(int dtype, int64_t K, int64_t M, int64_t row0, int64_t nrows, uint8_t * nat, uint8_t * rep, bool pack,
                           hipStream_t stream);

// bit-exact dequantization of n_blocks contiguous natural blocks into floats
hipError_t launch_dequantize(int dtype, const uint8_t * src, float * dst, int64_t n_blocks, hipStream_t stream);

// bit-exact (reference-identical) quantization of n_blocks blocks of floats into natural blocks
hipError_t launch_quantize(int dtype, const float * src, uint8_t * dst, int64_t n_blocks, hipStream_t stream);

// mean + stddev * N(0,1) with a counter-based generator (element i of stream seed uses counter i)
hipError_t launch_fill_normal(float * dst, int64_t n, uint64_t seed, float mean, float stddev, hipStream_t stream);

} // namespace sgk
