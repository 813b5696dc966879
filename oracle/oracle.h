/* CPU oracle for the quantized MUL_MAT path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU implementation (src/core/ref/f16.cpp,
 * src/core/ref/quant.cpp, src/core/ref/ops.cpp:32-41,78-93,258-269,690-721,802-1024) and of the R32 host pack/unpack
 * (src/backends/opencl11/r32.h:35-90, src/tensor/tensor.cpp:5-19). It is the checker of the GPU
 * path and the CPU baseline that bench.py times; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it. The product library never links or calls it.
 *
 * Status codes follow scrapgpu_status: 0 OK, 1 UNSUPPORTED, 2 INVALID_ARGUMENT. dtype values are
 * the scrapgpu_dtype enum values (F32 = 0, F16 = 1, BF16 = 5, Q4_0 = 16, Q8_0 = 17, Q4_K = 32,
 * Q6_K = 33). Float weights (F32, F16, BF16; MUL_MAT_ID and GET_ROWS: F32, F16) are read as the
 * reference's load_float reads them.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   half<->float         exhaustive half->float vs numpy; float->half RNE vs numpy on all
 *                        exponents + specials; reference bit patterns (ref_quant_tests.cpp:179-223)
 *   dequantize_*         reference hand-built blocks (ref_quant_tests.cpp:23-105) + golden vectors
 *                        produced by the reference compiled from source (tests/golden/)
 *   quantize_*           golden vectors from the compiled reference + round-trip bounds
 *                        (ref_quant_tests.cpp:112-158) + the cpu_bench checksums
 *   mul_mat              golden vectors (every weight dtype, float ones included), the
 *                        increasing-K cancellation case (ref_ops_tests.cpp:754-771), fp64 brute
 *                        force on small shapes, cpu_bench checksums (tools/cpu_bench.cpp)
 *   r32 pack/unpack      hand-checked layouts (r32_tests.cpp:104-181), pack/unpack identity,
 *                        golden vectors from the reference pack
 *   mul_mat_id           golden vectors from the compiled reference (scrapgpu_ref_execute), and
 *                        equality with per-pair mul_mat on the selected expert; out-of-range ids
 *   get_rows             golden vectors from the compiled reference, and equality with the
 *                        dequantized rows; out-of-range row indices
 */
#ifndef SGO_ORACLE_H
#define SGO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SGO_F32 = 0,
    SGO_F16 = 1,
    SGO_I32 = 2,
    SGO_BF16 = 5,
    SGO_Q4_0 = 16,
    SGO_Q8_0 = 17,
    SGO_Q4_K = 32,
    SGO_Q6_K = 33,
};

/* a host tensor: ggml orientation, byte strides, data points at element (0,0,0,0) */
typedef struct sgo_tensor {
    int32_t dtype;
    int64_t ne[4];
    uint64_t nb[4];
    void * data;
} sgo_tensor;

float sgo_half_to_float(uint16_t h);
uint16_t sgo_float_to_half(float f);
void sgo_half_to_float_n(const uint16_t * src, float * dst, int64_t n);
void sgo_float_to_half_n(const float * src, uint16_t * dst, int64_t n);

size_t sgo_block_size(int32_t dtype);
size_t sgo_type_size(int32_t dtype);

int sgo_dequantize(int32_t dtype, const void * src, float * dst, int64_t n);
int sgo_quantize(int32_t dtype, const float * src, void * dst, int64_t n);

/* dst = src0^T-product of exec_mul_mat: dst[m, n, i2, i3] = sum_k W[k, m, i2/r2, i3/r3] * x[k, n, i2, i3],
 * accumulated in float in increasing k, one multiply then one add per term. */
int sgo_mul_mat(const sgo_tensor * w, const sgo_tensor * x, sgo_tensor * y, int allow_broadcast);

/* Same, but the M rows of every slice are split over `threads` POSIX threads (an all-core variant
 * of the baseline; identical results). */
int sgo_mul_mat_mt(const sgo_tensor * w, const sgo_tensor * x, sgo_tensor * y, int allow_broadcast, int threads);

/* MUL_MAT_ID of ops.cpp:986-1024: dst[:, i, t] = w[:, :, ids[i, t]] x[:, i or 0, t] (scalar loop);
 * SGO_INVALID for an expert index outside [0, E). */
int sgo_mul_mat_id(const sgo_tensor * w, const sgo_tensor * x, const sgo_tensor * ids, sgo_tensor * y);

/* GET_ROWS of ops.cpp:690-721: dst[:, a, b, c] = dequantized row ids[a, b, c] of slice (b, c). */
int sgo_get_rows(const sgo_tensor * w, const sgo_tensor * ids, sgo_tensor * y);

/* R32 pack / unpack of `slices` contiguous slices of M rows of K elements (natural <-> repacked). */
int sgo_r32_pack(int32_t dtype, int64_t K, int64_t M, int64_t slices, const uint8_t * nat, uint8_t * rep);
int sgo_r32_unpack(int32_t dtype, int64_t K, int64_t M, int64_t slices, const uint8_t * rep, uint8_t * nat);

#ifdef __cplusplus
}
#endif

#endif
