/* The MI355X (gfx950) `hip` backend of ScrapGpuLibrary.
 *
 * Registration is the drop-in entry point; it sits beside the reference's
 * scrapgpu_opencl11_register (include/scrapgpu/opencl11.h:13, src/backends/opencl11/api.cpp:1477-1498).
 * The other functions are extensions with no counterpart in the reference's public headers; each
 * comment names what it stands in for. All of them report errors through scrapgpu_status and
 * scrapgpu_last_error() like the rest of the API. */
#ifndef SCRAPGPU_HIP_H
#define SCRAPGPU_HIP_H

#include "scrapgpu/backend.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Registers the hip backend: one device per visible AMD GPU of architecture gfx950
 * (SCRAPGPU_HIP_DEVICES="0,2" restricts the list). Safe to call more than once. Replaces
 * scrapgpu_opencl11_register (reference include/scrapgpu/opencl11.h:13). */
SCRAPGPU_API scrapgpu_status scrapgpu_hip_register(void);

/* Quantizes the F32 tensor `src` into the quantized tensor `dst` on the device (NATURAL or R32
 * layout, Q4_0 / Q8_0 / Q4_K / Q6_K). The bytes are identical to the reference quantizer's
 * (reference include/scrapgpu/reference.h:43, src/core/ref/quant.cpp:111-470) run on the same
 * values; here the data never leaves HBM. Both tensors must be contiguous and have the same shape. */
SCRAPGPU_API scrapgpu_status scrapgpu_hip_quantize(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * src, const scrapgpu_tensor_desc * dst);

/* Dequantizes the quantized tensor `src` (NATURAL or R32) into the F32 tensor `dst` on the device,
 * bit-identical to the reference's scrapgpu_ref_dequantize (reference.h:41,
 * src/core/ref/quant.cpp:30-108). Both tensors must be contiguous and have the same shape. */
SCRAPGPU_API scrapgpu_status scrapgpu_hip_dequantize(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * src, const scrapgpu_tensor_desc * dst);

/* Fills the contiguous F32 tensor `desc` with mean + stddev * N(0,1) samples: a counter-based
 * splitmix64 stream (element i of stream `seed` uses counter i) through Box-Muller. Synthetic
 * input generation for benchmarks; no counterpart in the reference. */
SCRAPGPU_API scrapgpu_status scrapgpu_hip_fill_normal(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * desc, uint64_t seed, float mean, float stddev);

/* Per-kernel timing, the counterpart of the reference's GGML_CL11_PROFILE table
 * (src/backends/opencl11/executor.h:41-131). While enabled every kernel launch of the backend is
 * bracketed by HIP events on the stream it runs on; scrapgpu_hip_profile_read synchronizes the
 * device and returns entry `index` (kernel name, launch count, summed milliseconds, summed
 * algorithmic bytes and flops); it returns SCRAPGPU_STATUS_INVALID_ARGUMENT past the last entry.
 * The environment variable SCRAPGPU_HIP_PROFILE=1 enables it at registration. */
SCRAPGPU_API scrapgpu_status scrapgpu_hip_profile_enable(int enable);
SCRAPGPU_API scrapgpu_status scrapgpu_hip_profile_reset(void);
SCRAPGPU_API scrapgpu_status scrapgpu_hip_profile_read(size_t index, const char ** name, uint64_t * launches, double * total_ms,
                                                      double * bytes, double * flops);

/* scrapgpu_op_execute for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * It runs the same kernels as scrapgpu_op_execute, but the scratch those kernels need (the prefill
 * GEMM's f16 activations and split-K partial sums, the grouped MUL_MAT_ID's routing tables, the
 * decode matvec's x planes and K-chunk partial sums) comes from a static array of 32 MiB per GPU
 * that the library holds until the process ends, instead of the stream's scratch, which
 * scrapgpu_op_execute grows with hipMalloc; it calls no hipMalloc or hipFree, and the event
 * profiler stays off during the call. One exception to "the same kernels": a prefill shape that
 * scrapgpu_op_execute runs in a stream-K form (its 384-row tiles fewer than the CUs, or a second
 * round of them at most a quarter full, and a long K) runs
 * another GEMM form here, whose output differs in rounding (both within the prefill tolerance),
 * because stream-K's partial slots do not fit the static array. An op that needs more than 32 MiB
 * of scratch is refused with SCRAPGPU_STATUS_UNSUPPORTED and a reason (decode matvecs need at most
 * a few MiB; prefill needs about 2 * N * K bytes plus, for split-K shapes, 4 * splits * N * M bytes).
 * Every call on one GPU shares that GPU's array: calls whose work overlaps on one GPU (two
 * streams, two threads) race on it; serialize them. */
SCRAPGPU_API scrapgpu_status scrapgpu_hip_op_execute_static(scrapgpu_stream_t * stream, const scrapgpu_op_desc * desc);

/* The kernel form (a short text such as "burst rg=3 W=4 spw=2" or "gemm w=12 kg=1 bn=64 rg=1
 * split=1") and work-group count of the calling thread's last matvec / matmul launch, for tests
 * that pin which kernel a shape selects. `form` receives at most `capacity` bytes including the
 * terminating NUL. Diagnostic extension; no counterpart in the reference. */
SCRAPGPU_API scrapgpu_status scrapgpu_hip_last_launch(char * form, size_t capacity, uint64_t * grid);

/* The native hipStream_t of a hip-backend stream (for callers that interoperate with other HIP
 * code); NULL for a stream of another backend. */
SCRAPGPU_API void * scrapgpu_hip_stream_native(scrapgpu_stream_t * stream);

#ifdef __cplusplus
}
#endif

#endif
