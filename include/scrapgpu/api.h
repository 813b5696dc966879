/* Public C ABI of ScrapGpuLibrary as implemented by this library (core + the MI355X `hip` backend).
 *
 * The layouts and enum values in these headers are the ABI of the reference's
 * include/scrapgpu/api.h:1-37 and must stay bit-identical so that callers built against the
 * reference headers can link against this library unchanged. */
#ifndef SCRAPGPU_API_H
#define SCRAPGPU_API_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define SCRAPGPU_API __attribute__((visibility("default")))
#else
#define SCRAPGPU_API
#endif

/* ABI 0.4 (reference api.h:19-20) */
#define SCRAPGPU_ABI_VERSION_MAJOR 0u
#define SCRAPGPU_ABI_VERSION_MINOR 4u

#ifdef __cplusplus
extern "C" {
#endif

typedef struct scrapgpu_device scrapgpu_device_t;
typedef struct scrapgpu_buffer scrapgpu_buffer_t;
typedef struct scrapgpu_stream scrapgpu_stream_t;
typedef struct scrapgpu_plan scrapgpu_plan_t;

/* (major << 16) | minor -- replaces reference src/core/status.cpp:11-13 */
SCRAPGPU_API uint32_t scrapgpu_get_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif
