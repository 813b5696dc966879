// Backend registry and object dispatch (reference src/core/registry.cpp:1-228).
//
// Every object handed out by a backend begins with a scrapgpu_object_header; the entry points
// below find the owning vtable through it and forward the call. A missing vtable entry is
// UNSUPPORTED with a reason; a foreign object is INVALID_ARGUMENT.
#include "scrapgpu/backend.h"
#include "scrapgpu/stream.h"


#include <algorithm>
#include <cstring>
#include <mutex>
#include <utility>
#include <vector>

namespace {

std::mutex g_mu;
std::vector<scrapgpu_backend_vtable> g_tables;

scrapgpu_status fail(scrapgpu_status st, const char * msg) {
    scrapgpu_set_last_error(msg);
    return st;
}

const scrapgpu_backend_vtable * owner(const void * obj) {
    return obj ? static_cast<const scrapgpu_object_header *>(obj)->backend : nullptr;
}

template <typename Fn, typename... Args>
scrapgpu_status forward(const void * obj, Fn scrapgpu_backend_vtable::*slot, const char * missing, Args &&... args) {
    const scrapgpu_backend_vtable * vt = owner(obj);
    if (vt == nullptr) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "object does not belong to a registered backend");
    if (vt->*slot == nullptr) return fail(SCRAPGPU_STATUS_UNSUPPORTED, missing);
    return (vt->*slot)(std::forward<Args>(args)...);
}

} // namespace

extern "C" {

scrapgpu_status scrapgpu_device_info_init(scrapgpu_device_info * info, size_t struct_size) {
    if (info == nullptr || struct_size < sizeof(size_t)) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "device info struct is too small");
    std::memset(info, 0, std::min(struct_size, sizeof(scrapgpu_device_info)));
    info->struct_size = struct_size;
    if (struct_size >= offsetof(scrapgpu_device_info, generation) + sizeof(info->generation)) {
        info->generation = SCRAPGPU_DEVICE_GENERATION_UNKNOWN;
    }
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status scrapgpu_register_backend(const scrapgpu_backend_vtable * vt) {
    if (vt == nullptr || vt->name == nullptr ||
        vt->struct_size < offsetof(scrapgpu_backend_vtable, plan_free) + sizeof(vt->plan_free)) {
        return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "backend vtable is incomplete");
    }
    scrapgpu_backend_vtable copy;
    std::memset(&copy, 0, sizeof(copy));
    std::memcpy(&copy, vt, std::min(vt->struct_size, sizeof(copy)));
    copy.struct_size = sizeof(copy);
    std::lock_guard<std::mutex> lock(g_mu);
    g_tables.push_back(copy);
    return SCRAPGPU_STATUS_OK;
}

void scrapgpu_unregister_all_backends(void) {
    std::lock_guard<std::mutex> lock(g_mu);
    g_tables.clear();
}

size_t scrapgpu_get_device_count(void) {
    std::lock_guard<std::mutex> lock(g_mu);
    size_t n = 0;
    for (const auto & t : g_tables)
        if (t.get_device_count) n += t.get_device_count(t.userdata);
    return n;
}

scrapgpu_status scrapgpu_get_device(size_t index, scrapgpu_device_t ** out) {
    if (out == nullptr) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "out_device is null");
    std::lock_guard<std::mutex> lock(g_mu);
    for (const auto & t : g_tables) {
        if (!t.get_device_count || !t.get_device) continue;
        const size_t n = t.get_device_count(t.userdata);
        if (index < n) return t.get_device(t.userdata, index, out);
        index -= n;
    }
    *out = nullptr;
    return fail(SCRAPGPU_STATUS_UNSUPPORTED, "no backend device at the requested index");
}

scrapgpu_status scrapgpu_device_get_info(scrapgpu_device_t * device, scrapgpu_device_info * info) {
    if (device == nullptr || info == nullptr) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "device or info is null");
    return forward(device, &scrapgpu_backend_vtable::device_get_info, "the backend cannot describe the device", device, info);
}

scrapgpu_status scrapgpu_buffer_alloc(scrapgpu_device_t * device, size_t size, scrapgpu_buffer_t ** out) {
    if (device == nullptr || out == nullptr) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "device or out_buffer is null");
    *out = nullptr;
    return forward(device, &scrapgpu_backend_vtable::buffer_alloc, "the device backend cannot allocate buffers", device, size, out);
}

scrapgpu_status scrapgpu_buffer_free(scrapgpu_buffer_t * buffer) {
    if (buffer == nullptr) return SCRAPGPU_STATUS_OK;
    return forward(buffer, &scrapgpu_backend_vtable::buffer_free, "the buffer backend cannot free buffers", buffer);
}

scrapgpu_status scrapgpu_buffer_write(scrapgpu_stream_t * s, scrapgpu_buffer_t * b, uint64_t off, const void * data, size_t size, int blocking) {
    if (s == nullptr || b == nullptr || (data == nullptr && size != 0)) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "stream, buffer or data is null");
    return forward(s, &scrapgpu_backend_vtable::buffer_write, "the stream backend cannot write buffers", s, b, off, data, size, blocking);
}

scrapgpu_status scrapgpu_buffer_read(scrapgpu_stream_t * s, scrapgpu_buffer_t * b, uint64_t off, void * data, size_t size, int blocking) {
    if (s == nullptr || b == nullptr || (data == nullptr && size != 0)) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "stream, buffer or data is null");
    return forward(s, &scrapgpu_backend_vtable::buffer_read, "the stream backend cannot read buffers", s, b, off, data, size, blocking);
}

scrapgpu_status scrapgpu_buffer_copy(scrapgpu_stream_t * s, scrapgpu_buffer_t * dst, uint64_t doff, scrapgpu_buffer_t * src, uint64_t soff, size_t size, int blocking) {
    if (s == nullptr || dst == nullptr || src == nullptr) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "stream, dst or src is null");
    return forward(s, &scrapgpu_backend_vtable::buffer_copy, "the stream backend cannot copy buffers", s, dst, doff, src, soff, size, blocking);
}

scrapgpu_status scrapgpu_buffer_fill(scrapgpu_stream_t * s, scrapgpu_buffer_t * b, uint64_t off, size_t size, uint8_t byte, int blocking) {
    if (s == nullptr || b == nullptr) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "stream or buffer is null");
    return forward(s, &scrapgpu_backend_vtable::buffer_fill, "the stream backend cannot fill buffers", s, b, off, size, byte, blocking);
}

scrapgpu_status scrapgpu_stream_create(scrapgpu_device_t * device, scrapgpu_stream_t ** out) {
    if (device == nullptr || out == nullptr) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "device or out_stream is null");
    *out = nullptr;
    return forward(device, &scrapgpu_backend_vtable::stream_create, "the device backend cannot create streams", device, out);
}

scrapgpu_status scrapgpu_stream_free(scrapgpu_stream_t * s) {
    if (s == nullptr) return SCRAPGPU_STATUS_OK;
    return forward(s, &scrapgpu_backend_vtable::stream_free, "the stream backend cannot free streams", s);
}

scrapgpu_status scrapgpu_stream_sync(scrapgpu_stream_t * s) {
    if (s == nullptr) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "stream is null");
    return forward(s, &scrapgpu_backend_vtable::stream_sync, "the stream backend cannot synchronize", s);
}

scrapgpu_status scrapgpu_tensor_upload(scrapgpu_stream_t * s, const scrapgpu_tensor_desc * d, const void * host, size_t size) {
    if (s == nullptr || d == nullptr || (host == nullptr && size != 0)) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "stream, tensor desc or host pointer is null");
    return forward(s, &scrapgpu_backend_vtable::tensor_upload, "the stream backend cannot upload tensors", s, d, host, size);
}

scrapgpu_status scrapgpu_tensor_download(scrapgpu_stream_t * s, const scrapgpu_tensor_desc * d, void * host, size_t size) {
    if (s == nullptr || d == nullptr || (host == nullptr && size != 0)) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "stream, tensor desc or host pointer is null");
    return forward(s, &scrapgpu_backend_vtable::tensor_download, "the stream backend cannot download tensors", s, d, host, size);
}

scrapgpu_status scrapgpu_plan_build(scrapgpu_device_t * device, const scrapgpu_plan_desc * desc, scrapgpu_plan_t ** out) {
    if (device == nullptr || desc == nullptr || out == nullptr) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "device, plan desc, or out_plan is null");
    *out = nullptr;
    return forward(device, &scrapgpu_backend_vtable::plan_build, "the device backend cannot build plans", device, desc, out);
}

scrapgpu_status scrapgpu_plan_execute(scrapgpu_stream_t * s, scrapgpu_plan_t * plan) {
    if (s == nullptr || plan == nullptr) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "stream or plan is null");
    if (owner(s) == nullptr || owner(s) != owner(plan)) return fail(SCRAPGPU_STATUS_INVALID_ARGUMENT, "stream and plan belong to different backends");
    return forward(s, &scrapgpu_backend_vtable::plan_execute, "the stream backend cannot execute plans", s, plan);
}

scrapgpu_status scrapgpu_plan_free(scrapgpu_plan_t * plan) {
    if (plan == nullptr) return SCRAPGPU_STATUS_OK;
    return forward(plan, &scrapgpu_backend_vtable::plan_free, "the plan backend cannot free plans", plan);
}

}
