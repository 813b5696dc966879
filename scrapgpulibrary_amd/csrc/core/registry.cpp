// Backend registration, device enumeration and routing of the object calls to their backend.
//
// Semantics follow the reference's vtable contract (include/scrapgpu/backend.h:29-59): a
// backend registers a table whose struct_size covers at least the ABI 0.2 entries (through
// plan_free) and has a name; device indices run over the backends in registration order; calls on
// a device, buffer, stream or plan go to the backend named by the object's header. A null
// required argument is INVALID_ARGUMENT, an entry the backend left null is UNSUPPORTED with a
// reason, and freeing a null object is a no-op. Registering a table that is already registered
// replaces its entry instead of listing its devices twice.
//
// The core calls through padded copies of the tables. A copy is never freed before the process
// ends, so a table pointer handed to a caller stays valid while another thread re-registers or
// unregisters. An object whose header names a table that is not (or no longer) registered is
// dispatched through a padded copy of that header's own table, as the reference dispatches through
// the header (src/core/registry.cpp): its buffers, streams and plans can still be used and freed
// after scrapgpu_unregister_all_backends.
#include "dispatch.h"
#include "scrapgpu/stream.h"

#include <algorithm>
#include <cstddef>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace {

struct Registered {
    const scrapgpu_backend_vtable * origin; // the table the backend passed (what headers point at)
    scrapgpu_backend_vtable table;          // the core's padded copy
};

constexpr size_t kMinTable = offsetof(scrapgpu_backend_vtable, plan_free) + sizeof(void (*)());

class Registry {
  public:
    static Registry & get() {
        static Registry r;
        return r;
    }

    void add(const scrapgpu_backend_vtable * vt) {
        std::lock_guard<std::mutex> hold(mu_);
        Registered * e = copy_of(vt);
        for (auto & old : list_) {
            if (old->origin == vt) {
                old = e;
                return;
            }
        }
        list_.push_back(e);
    }

    void clear() {
        std::lock_guard<std::mutex> hold(mu_);
        list_.clear();
    }

    // the table to call for objects whose header names `origin`: its registered copy, else the
    // latest copy made of it, else a new padded copy of it (null: not a usable table)
    const scrapgpu_backend_vtable * find(const scrapgpu_backend_vtable * origin) {
        if (origin == nullptr) return nullptr;
        std::lock_guard<std::mutex> hold(mu_);
        for (const Registered * e : list_)
            if (e->origin == origin) return &e->table;
        for (auto it = all_.rbegin(); it != all_.rend(); ++it)
            if ((*it)->origin == origin) return &(*it)->table;
        if (origin->struct_size < kMinTable || origin->name == nullptr) return nullptr;
        return &copy_of(origin)->table;
    }

    // calls fn(table) for each registered table, in registration order, until it returns true
    template <typename Fn>
    void each(Fn && fn) {
        std::lock_guard<std::mutex> hold(mu_);
        for (const Registered * e : list_)
            if (fn(e->table)) return;
    }

  private:
    // a new padded copy of vt, kept until the process ends (mu_ held)
    Registered * copy_of(const scrapgpu_backend_vtable * vt) {
        auto e = std::make_unique<Registered>();
        e->origin = vt;
        std::memset(&e->table, 0, sizeof(e->table));
        std::memcpy(&e->table, vt, std::min(vt->struct_size, sizeof(e->table)));
        e->table.struct_size = sizeof(e->table);
        all_.push_back(std::move(e));
        return all_.back().get();
    }

    std::mutex mu_;
    std::vector<std::unique_ptr<Registered>> all_; // every copy ever made
    std::vector<Registered *> list_;               // the registered ones, in registration order
};

scrapgpu_status complain(scrapgpu_status st, const std::string & msg) {
    scrapgpu_set_last_error(msg.c_str());
    return st;
}

} // namespace

namespace sgcore {

const scrapgpu_backend_vtable * owner_table(const void * obj, const char * call, const char * what) {
    const scrapgpu_backend_vtable * t = nullptr;
    if (obj != nullptr) t = Registry::get().find(static_cast<const scrapgpu_object_header *>(obj)->backend);
    if (t == nullptr) complain(SCRAPGPU_STATUS_INVALID_ARGUMENT, std::string(call) + ": " + what + " is not an object of a backend (no usable table in its header)");
    return t;
}

scrapgpu_status null_argument(const char * call, const char * what) {
    return complain(SCRAPGPU_STATUS_INVALID_ARGUMENT, std::string(call) + ": " + what + " is null");
}

scrapgpu_status not_implemented(const char * call, const scrapgpu_backend_vtable * table, const char * entry) {
    return complain(SCRAPGPU_STATUS_UNSUPPORTED, std::string(call) + ": backend '" + (table->name ? table->name : "?") +
                                                     "' does not implement " + entry);
}

} // namespace sgcore

using sgcore::not_implemented;
using sgcore::null_argument;
using sgcore::owner_table;

extern "C" {

scrapgpu_status scrapgpu_device_info_init(scrapgpu_device_info * info, size_t struct_size) {
    const char * call = "scrapgpu_device_info_init";
    if (info == nullptr) return null_argument(call, "info");
    if (struct_size < sizeof(info->struct_size)) return complain(SCRAPGPU_STATUS_INVALID_ARGUMENT, std::string(call) + ": struct_size cannot hold the size field");
    std::memset(info, 0, std::min(struct_size, sizeof(*info)));
    info->struct_size = struct_size;
    if (struct_size >= offsetof(scrapgpu_device_info, generation) + sizeof(info->generation)) info->generation = SCRAPGPU_DEVICE_GENERATION_UNKNOWN;
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status scrapgpu_register_backend(const scrapgpu_backend_vtable * backend) {
    const char * call = "scrapgpu_register_backend";
    if (backend == nullptr) return null_argument(call, "backend");
    if (backend->struct_size < kMinTable) return complain(SCRAPGPU_STATUS_INVALID_ARGUMENT, std::string(call) + ": struct_size is below the ABI 0.2 table");
    if (backend->name == nullptr) return complain(SCRAPGPU_STATUS_INVALID_ARGUMENT, std::string(call) + ": the table has no name");
    Registry::get().add(backend);
    return SCRAPGPU_STATUS_OK;
}

void scrapgpu_unregister_all_backends(void) {
    Registry::get().clear();
}

size_t scrapgpu_get_device_count(void) {
    size_t total = 0;
    Registry::get().each([&](const scrapgpu_backend_vtable & t) {
        if (t.get_device_count != nullptr) total += t.get_device_count(t.userdata);
        return false;
    });
    return total;
}

scrapgpu_status scrapgpu_get_device(size_t index, scrapgpu_device_t ** out_device) {
    const char * call = "scrapgpu_get_device";
    if (out_device == nullptr) return null_argument(call, "out_device");
    *out_device = nullptr;
    scrapgpu_status st = SCRAPGPU_STATUS_UNSUPPORTED;
    bool found = false;
    size_t left = index;
    Registry::get().each([&](const scrapgpu_backend_vtable & t) {
        const size_t n = t.get_device_count != nullptr && t.get_device != nullptr ? t.get_device_count(t.userdata) : 0;
        if (left >= n) {
            left -= n;
            return false;
        }
        found = true;
        st = t.get_device(t.userdata, left, out_device);
        return true;
    });
    if (!found) return complain(SCRAPGPU_STATUS_UNSUPPORTED, std::string(call) + ": index " + std::to_string(index) + " is past the last device");
    return st;
}

scrapgpu_status scrapgpu_device_get_info(scrapgpu_device_t * device, scrapgpu_device_info * info) {
    const char * call = "scrapgpu_device_get_info";
    if (info == nullptr) return null_argument(call, "info");
    const scrapgpu_backend_vtable * t = owner_table(device, call, "device");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->device_get_info == nullptr) return not_implemented(call, t, "device_get_info");
    return t->device_get_info(device, info);
}

scrapgpu_status scrapgpu_buffer_alloc(scrapgpu_device_t * device, size_t size, scrapgpu_buffer_t ** out_buffer) {
    const char * call = "scrapgpu_buffer_alloc";
    if (out_buffer == nullptr) return null_argument(call, "out_buffer");
    *out_buffer = nullptr;
    const scrapgpu_backend_vtable * t = owner_table(device, call, "device");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->buffer_alloc == nullptr) return not_implemented(call, t, "buffer_alloc");
    return t->buffer_alloc(device, size, out_buffer);
}

scrapgpu_status scrapgpu_buffer_free(scrapgpu_buffer_t * buffer) {
    const char * call = "scrapgpu_buffer_free";
    if (buffer == nullptr) return SCRAPGPU_STATUS_OK;
    const scrapgpu_backend_vtable * t = owner_table(buffer, call, "buffer");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->buffer_free == nullptr) return not_implemented(call, t, "buffer_free");
    return t->buffer_free(buffer);
}

scrapgpu_status scrapgpu_buffer_write(scrapgpu_stream_t * stream, scrapgpu_buffer_t * buffer, uint64_t offset, const void * data, size_t size,
                                      int blocking) {
    const char * call = "scrapgpu_buffer_write";
    if (buffer == nullptr) return null_argument(call, "buffer");
    if (data == nullptr && size != 0) return null_argument(call, "data");
    const scrapgpu_backend_vtable * t = owner_table(stream, call, "stream");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->buffer_write == nullptr) return not_implemented(call, t, "buffer_write");
    return t->buffer_write(stream, buffer, offset, data, size, blocking);
}

scrapgpu_status scrapgpu_buffer_read(scrapgpu_stream_t * stream, scrapgpu_buffer_t * buffer, uint64_t offset, void * data, size_t size, int blocking) {
    const char * call = "scrapgpu_buffer_read";
    if (buffer == nullptr) return null_argument(call, "buffer");
    if (data == nullptr && size != 0) return null_argument(call, "data");
    const scrapgpu_backend_vtable * t = owner_table(stream, call, "stream");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->buffer_read == nullptr) return not_implemented(call, t, "buffer_read");
    return t->buffer_read(stream, buffer, offset, data, size, blocking);
}

scrapgpu_status scrapgpu_buffer_copy(scrapgpu_stream_t * stream, scrapgpu_buffer_t * dst, uint64_t dst_offset, scrapgpu_buffer_t * src,
                                     uint64_t src_offset, size_t size, int blocking) {
    const char * call = "scrapgpu_buffer_copy";
    if (dst == nullptr) return null_argument(call, "dst");
    if (src == nullptr) return null_argument(call, "src");
    const scrapgpu_backend_vtable * t = owner_table(stream, call, "stream");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->buffer_copy == nullptr) return not_implemented(call, t, "buffer_copy");
    return t->buffer_copy(stream, dst, dst_offset, src, src_offset, size, blocking);
}

scrapgpu_status scrapgpu_buffer_fill(scrapgpu_stream_t * stream, scrapgpu_buffer_t * buffer, uint64_t offset, size_t size, uint8_t byte, int blocking) {
    const char * call = "scrapgpu_buffer_fill";
    if (buffer == nullptr) return null_argument(call, "buffer");
    const scrapgpu_backend_vtable * t = owner_table(stream, call, "stream");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->buffer_fill == nullptr) return not_implemented(call, t, "buffer_fill");
    return t->buffer_fill(stream, buffer, offset, size, byte, blocking);
}

scrapgpu_status scrapgpu_stream_create(scrapgpu_device_t * device, scrapgpu_stream_t ** out_stream) {
    const char * call = "scrapgpu_stream_create";
    if (out_stream == nullptr) return null_argument(call, "out_stream");
    *out_stream = nullptr;
    const scrapgpu_backend_vtable * t = owner_table(device, call, "device");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->stream_create == nullptr) return not_implemented(call, t, "stream_create");
    return t->stream_create(device, out_stream);
}

scrapgpu_status scrapgpu_stream_free(scrapgpu_stream_t * stream) {
    const char * call = "scrapgpu_stream_free";
    if (stream == nullptr) return SCRAPGPU_STATUS_OK;
    const scrapgpu_backend_vtable * t = owner_table(stream, call, "stream");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->stream_free == nullptr) return not_implemented(call, t, "stream_free");
    return t->stream_free(stream);
}

scrapgpu_status scrapgpu_stream_sync(scrapgpu_stream_t * stream) {
    const char * call = "scrapgpu_stream_sync";
    if (stream == nullptr) return null_argument(call, "stream");
    const scrapgpu_backend_vtable * t = owner_table(stream, call, "stream");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->stream_sync == nullptr) return not_implemented(call, t, "stream_sync");
    return t->stream_sync(stream);
}

scrapgpu_status scrapgpu_tensor_upload(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * desc, const void * host, size_t size) {
    const char * call = "scrapgpu_tensor_upload";
    if (desc == nullptr) return null_argument(call, "desc");
    if (host == nullptr && size != 0) return null_argument(call, "host");
    const scrapgpu_backend_vtable * t = owner_table(stream, call, "stream");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->tensor_upload == nullptr) return not_implemented(call, t, "tensor_upload");
    return t->tensor_upload(stream, desc, host, size);
}

scrapgpu_status scrapgpu_tensor_download(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * desc, void * host, size_t size) {
    const char * call = "scrapgpu_tensor_download";
    if (desc == nullptr) return null_argument(call, "desc");
    if (host == nullptr && size != 0) return null_argument(call, "host");
    const scrapgpu_backend_vtable * t = owner_table(stream, call, "stream");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->tensor_download == nullptr) return not_implemented(call, t, "tensor_download");
    return t->tensor_download(stream, desc, host, size);
}

scrapgpu_status scrapgpu_plan_build(scrapgpu_device_t * device, const scrapgpu_plan_desc * desc, scrapgpu_plan_t ** out_plan) {
    const char * call = "scrapgpu_plan_build";
    if (desc == nullptr) return null_argument(call, "desc");
    if (out_plan == nullptr) return null_argument(call, "out_plan");
    *out_plan = nullptr;
    const scrapgpu_backend_vtable * t = owner_table(device, call, "device");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->plan_build == nullptr) return not_implemented(call, t, "plan_build");
    return t->plan_build(device, desc, out_plan);
}

scrapgpu_status scrapgpu_plan_execute(scrapgpu_stream_t * stream, scrapgpu_plan_t * plan) {
    const char * call = "scrapgpu_plan_execute";
    const scrapgpu_backend_vtable * t = owner_table(stream, call, "stream");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    const scrapgpu_backend_vtable * tp = owner_table(plan, call, "plan");
    if (tp == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (tp != t) return complain(SCRAPGPU_STATUS_INVALID_ARGUMENT, std::string(call) + ": the plan was built by backend '" + tp->name +
                                                                       "', the stream is of backend '" + t->name + "'");
    if (t->plan_execute == nullptr) return not_implemented(call, t, "plan_execute");
    return t->plan_execute(stream, plan);
}

scrapgpu_status scrapgpu_plan_free(scrapgpu_plan_t * plan) {
    const char * call = "scrapgpu_plan_free";
    if (plan == nullptr) return SCRAPGPU_STATUS_OK;
    const scrapgpu_backend_vtable * t = owner_table(plan, call, "plan");
    if (t == nullptr) return SCRAPGPU_STATUS_INVALID_ARGUMENT;
    if (t->plan_free == nullptr) return not_implemented(call, t, "plan_free");
    return t->plan_free(plan);
}

} // extern "C"
