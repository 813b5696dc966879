/* In-order execution queues (reference include/scrapgpu/stream.h). Work is enqueued
 * asynchronously; scrapgpu_stream_sync waits for everything submitted so far and reports kernel
 * failures that surfaced since the previous sync. A stream is used from one thread at a time. */
#ifndef SCRAPGPU_STREAM_H
#define SCRAPGPU_STREAM_H

#include "scrapgpu/device.h"

#ifdef __cplusplus
extern "C" {
#endif

SCRAPGPU_API scrapgpu_status scrapgpu_stream_create(scrapgpu_device_t * device, scrapgpu_stream_t ** out_stream);
SCRAPGPU_API scrapgpu_status scrapgpu_stream_free(scrapgpu_stream_t * stream);
SCRAPGPU_API scrapgpu_status scrapgpu_stream_sync(scrapgpu_stream_t * stream);

#ifdef __cplusplus
}
#endif

#endif
