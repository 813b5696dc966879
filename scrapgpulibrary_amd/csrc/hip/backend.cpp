// The `hip` backend: the scrapgpu_backend_vtable of one process over the visible gfx950 GPUs.
//
// Replaces, for the quantized MUL_MAT path, what the reference's OpenCL backend does in
// src/backends/opencl11/api.cpp (objects :45-79, support :252-258,467-473, resolve :546,
// dispatch :738-773, transfers :1234-1287, plans :1335-1443, vtable :1449-1473, registration
// :1477-1498) -- redesigned around HIP: one hipStream_t per scrapgpu stream, hipMalloc'd buffers,
// R32 packing done by a kernel in HBM instead of on the host, and kernel selection by shape
// (N <= 8: decode matvec; N > 8: f16 MFMA prefill).
#include "scrapgpu/hip.h"

#include "../core/tensor_math.h"
#include "kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace {

extern const scrapgpu_backend_vtable kVtable;

// ---- errors -------------------------------------------------------------------------------------

scrapgpu_status set_err(scrapgpu_status st, const std::string & msg) {
    scrapgpu_set_last_error(msg.c_str());
    return st;
}

scrapgpu_status invalid(const char * m) {
    return set_err(SCRAPGPU_STATUS_INVALID_ARGUMENT, m);
}

scrapgpu_status unsupported(const char * m, const char ** reason = nullptr) {
    if (reason) *reason = m;
    return set_err(SCRAPGPU_STATUS_UNSUPPORTED, m);
}

scrapgpu_status hip_fail(hipError_t e, const char * what) {
    const std::string msg = std::string(what) + ": " + hipGetErrorString(e);
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) return set_err(SCRAPGPU_STATUS_OUT_OF_MEMORY, msg);
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice || e == hipErrorLaunchFailure || e == hipErrorIllegalAddress) {
        return set_err(SCRAPGPU_STATUS_DEVICE_LOST, msg);
    }
    return set_err(SCRAPGPU_STATUS_BACKEND_ERROR, msg);
}

#define SG_HIP(expr, what)                          \
    do {                                            \
        const hipError_t e_ = (expr);               \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

// ---- objects --------------------------------------------------------------------------------------

struct Device;

struct Buffer {
    scrapgpu_object_header hdr;
    Device * dev;
    uint8_t * ptr;
    size_t size;
    std::atomic<int> plan_refs{0};
};

struct Stream {
    scrapgpu_object_header hdr;
    Device * dev;
    hipStream_t s;
    uint8_t * scratch = nullptr; // prefill matmul: f16 activations, row factors and split-K partials (grown on demand)
    size_t scratch_size = 0;
    uint64_t scratch_gen = 0;    // process-unique: set at creation, renewed on every re-allocation (keys recorded graphs)
    uint32_t * arrive = nullptr; // the chunked decode matvec's arrival counts (sgk::kArriveMax, zero between launches)
};

std::atomic<uint64_t> g_scratch_gen{1};

struct Device {
    scrapgpu_object_header hdr;
    int ordinal;
    std::string name, arch, driver, tuning;
    uint64_t total_mem = 0;
    uint64_t lds = 0;
    uint32_t cus = 0;
    std::mutex mu;          // guards the staging buffer and the profiling records
    uint8_t * staging = nullptr;
    size_t staging_size = 0;
    uint8_t * static_scratch = nullptr; // this device's copy of `scratch` (below), or null
    uint32_t * static_arrive = nullptr; // this device's copy of `arrive_counts` (below), or null
};

struct PlanNode {
    scrapgpu_op_desc op;
    std::vector<scrapgpu_tensor_desc> in, out;
    std::vector<uint8_t> params;
    int fuse = 0; // the next `fuse` nodes run in this node's launch (MUL_MAT_ID sharing x and ids)
};

struct Plan {
    scrapgpu_object_header hdr;
    Device * dev;
    std::vector<PlanNode> nodes;
    std::vector<Buffer *> buffers;
    // the launches of all nodes recorded once as a HIP graph and replayed (per stream: the
    // kernels use the recording stream's scratch)
    // the captured graph is kept as long as its instantiation (a tracer that resolves a launch's
    // nodes through the source graph finds it alive)
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    Stream * exec_stream = nullptr;
    uint64_t exec_gen = 0;
};

struct Registry {
    std::mutex mu;
    bool registered = false;
    std::vector<std::unique_ptr<Device>> devices;
};

Registry & registry() {
    static Registry r;
    return r;
}

template <typename T>
T * as(void * obj) {
    T * t = static_cast<T *>(obj);
    return t != nullptr && t->hdr.backend == &kVtable ? t : nullptr;
}

Device * dev_of(scrapgpu_device_t * d) {
    return as<Device>(d);
}
Buffer * buf_of(scrapgpu_buffer_t * b) {
    return as<Buffer>(b);
}
Stream * stream_of(scrapgpu_stream_t * s) {
    return as<Stream>(s);
}

hipError_t use(Device * d) {
    return hipSetDevice(d->ordinal);
}

// ---- profiling (per-launch HIP events) ----------------------------------------------------------

struct ProfRecord {
    std::string name;
    hipEvent_t a, b;
    double bytes, flops;
};

struct ProfEntry {
    std::string name;
    uint64_t launches = 0;
    double ms = 0, bytes = 0, flops = 0;
};

std::atomic<bool> g_prof{false};
// while a scrapgpu_hip_op_execute_static call runs on this thread: its device's static scratch
// (the profiler stays off then: its events are allocations)
thread_local uint8_t * t_static_scratch = nullptr;
thread_local uint32_t * t_static_arrive = nullptr;
std::mutex g_prof_mu;
std::vector<ProfRecord> g_prof_pending;
std::vector<ProfEntry> g_prof_table;

struct ProfScope {
    hipStream_t s;
    const char * name = nullptr;
    double bytes = 0, flops = 0;
    hipEvent_t a = nullptr, b = nullptr;
    explicit ProfScope(hipStream_t st) : s(st) {
        if (g_prof.load(std::memory_order_relaxed) && t_static_scratch == nullptr && hipEventCreate(&a) == hipSuccess && hipEventCreate(&b) == hipSuccess) {
            hipEventRecord(a, s);
        } else {
            a = b = nullptr;
        }
    }
    void done(const char * n, double by, double fl) {
        if (a == nullptr) return;
        hipEventRecord(b, s);
        std::lock_guard<std::mutex> lock(g_prof_mu);
        g_prof_pending.push_back({n ? n : "kernel", a, b, by, fl});
        a = b = nullptr;
    }
    ~ProfScope() {
        if (a) hipEventDestroy(a);
        if (b) hipEventDestroy(b);
    }
};

void prof_collect() {
    std::lock_guard<std::mutex> lock(g_prof_mu);
    for (ProfRecord & r : g_prof_pending) {
        float ms = 0;
        hipEventSynchronize(r.b);
        hipEventElapsedTime(&ms, r.a, r.b);
        auto it = std::find_if(g_prof_table.begin(), g_prof_table.end(), [&](const ProfEntry & e) { return e.name == r.name; });
        if (it == g_prof_table.end()) {
            g_prof_table.push_back({r.name});
            it = g_prof_table.end() - 1;
        }
        it->launches += 1;
        it->ms += ms;
        it->bytes += r.bytes;
        it->flops += r.flops;
        hipEventDestroy(r.a);
        hipEventDestroy(r.b);
    }
    g_prof_pending.clear();
}

// ---- descriptors ----------------------------------------------------------------------------------

// a caller desc with a smaller struct_size: missing tail = buffer NULL, offset 0, NATURAL
scrapgpu_tensor_desc load_desc(const scrapgpu_tensor_desc & in) {
    scrapgpu_tensor_desc d;
    std::memset(&d, 0, sizeof(d));
    std::memcpy(&d, &in, std::min(in.struct_size, sizeof(d)));
    d.struct_size = sizeof(d);
    return d;
}

// the device address of a tensor after the bounds check against its buffer
scrapgpu_status resolve(Device * dev, const scrapgpu_tensor_desc & t, uint8_t ** out, const char * what) {
    Buffer * b = buf_of(t.buffer);
    if (b == nullptr) return set_err(SCRAPGPU_STATUS_INVALID_ARGUMENT, std::string(what) + " has no hip buffer");
    if (b->dev != dev) return set_err(SCRAPGPU_STATUS_INVALID_ARGUMENT, std::string(what) + " lives on another device");
    const uint64_t n = sg::nbytes(t);
    if (t.offset > b->size || n > b->size - t.offset) {
        return set_err(SCRAPGPU_STATUS_INVALID_ARGUMENT, std::string(what) + " reaches past the end of its buffer");
    }
    *out = b->ptr + t.offset;
    return SCRAPGPU_STATUS_OK;
}

// ---- device enumeration -----------------------------------------------------------------------

size_t api_device_count(void *) {
    std::lock_guard<std::mutex> lock(registry().mu);
    return registry().devices.size();
}

scrapgpu_status api_get_device(void *, size_t index, scrapgpu_device_t ** out) {
    std::lock_guard<std::mutex> lock(registry().mu);
    if (index >= registry().devices.size()) return invalid("no hip device has this index");
    *out = reinterpret_cast<scrapgpu_device_t *>(registry().devices[index].get());
    return SCRAPGPU_STATUS_OK;
}

#define SG_INFO_SET(field, value)                                                        \
    do {                                                                                 \
        if (info->struct_size >= offsetof(scrapgpu_device_info, field) + sizeof(info->field)) info->field = (value); \
    } while (0)

scrapgpu_status api_device_info(scrapgpu_device_t * device, scrapgpu_device_info * info) {
    Device * d = dev_of(device);
    if (d == nullptr) return invalid("not a hip device");
    if (info->struct_size < sizeof(size_t)) return invalid("the device info struct cannot hold its size field");
    SG_INFO_SET(name, d->name.c_str());
    SG_INFO_SET(vendor, "AMD");
    SG_INFO_SET(platform_name, "HIP");
    SG_INFO_SET(driver_version, d->driver.c_str());
    SG_INFO_SET(backend_name, "hip");
    SG_INFO_SET(reported_api_version, d->driver.c_str());
    SG_INFO_SET(used_api_version, d->driver.c_str());
    SG_INFO_SET(generation, SCRAPGPU_DEVICE_GENERATION_AMD_GCN);
    SG_INFO_SET(generation_reason, d->arch.c_str());
    SG_INFO_SET(total_memory_bytes, d->total_mem);
    SG_INFO_SET(max_allocation_reported_bytes, d->total_mem);
    SG_INFO_SET(max_allocation_used_bytes, d->total_mem);
    SG_INFO_SET(max_work_group_size, (uint64_t) 1024);
    SG_INFO_SET(local_memory_bytes, d->lds);
    SG_INFO_SET(compute_units, d->cus);
    SG_INFO_SET(warp_or_wave_width, 64u);
    SG_INFO_SET(quirks, (uint64_t) 0);
    SG_INFO_SET(probed_quirks, (uint64_t) 0);
    SG_INFO_SET(tuning_profile_name, d->tuning.c_str());
    SG_INFO_SET(tuning_overrides, "");
    return SCRAPGPU_STATUS_OK;
}

// ---- buffers --------------------------------------------------------------------------------------

scrapgpu_status api_buffer_alloc(scrapgpu_device_t * device, size_t size, scrapgpu_buffer_t ** out) {
    Device * d = dev_of(device);
    if (d == nullptr) return invalid("not a hip device");
    SG_HIP(use(d), "hipSetDevice");
    void * p = nullptr;
    SG_HIP(hipMalloc(&p, std::max<size_t>(size, 256)), "hipMalloc");
    Buffer * b = new Buffer;
    b->hdr.backend = &kVtable;
    b->dev = d;
    b->ptr = static_cast<uint8_t *>(p);
    b->size = size;
    *out = reinterpret_cast<scrapgpu_buffer_t *>(b);
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status api_buffer_free(scrapgpu_buffer_t * buffer) {
    Buffer * b = buf_of(buffer);
    if (b == nullptr) return invalid("not a hip buffer");
    if (b->plan_refs.load() > 0) return invalid("the buffer is referenced by a live plan");
    use(b->dev);
    // work that still reads the buffer must finish before the memory is returned
    hipDeviceSynchronize();
    const hipError_t e = hipFree(b->ptr);
    delete b;
    if (e != hipSuccess) return hip_fail(e, "hipFree");
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status check_range(Stream * s, Buffer * b, uint64_t off, size_t size) {
    if (s == nullptr || b == nullptr) return invalid("not a hip stream or buffer");
    if (b->dev != s->dev) return invalid("the buffer lives on another device than the stream");
    if (off > b->size || size > b->size - off) return invalid("range exceeds the buffer");
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status finish(Stream * s, int blocking, const char * what) {
    if (blocking) SG_HIP(hipStreamSynchronize(s->s), what);
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status api_buffer_write(scrapgpu_stream_t * stream, scrapgpu_buffer_t * buffer, uint64_t off, const void * data, size_t size, int blocking) {
    Stream * s = stream_of(stream);
    Buffer * b = buf_of(buffer);
    scrapgpu_status st = check_range(s, b, off, size);
    if (st != SCRAPGPU_STATUS_OK || size == 0) return st;
    SG_HIP(use(s->dev), "hipSetDevice");
    SG_HIP(hipMemcpyAsync(b->ptr + off, data, size, hipMemcpyHostToDevice, s->s), "hipMemcpyAsync");
    // the host pointer may be reused on return (as for the reference's blocking writes)
    return finish(s, 1, "buffer_write");
}

scrapgpu_status api_buffer_read(scrapgpu_stream_t * stream, scrapgpu_buffer_t * buffer, uint64_t off, void * data, size_t size, int blocking) {
    Stream * s = stream_of(stream);
    Buffer * b = buf_of(buffer);
    scrapgpu_status st = check_range(s, b, off, size);
    if (st != SCRAPGPU_STATUS_OK || size == 0) return st;
    SG_HIP(use(s->dev), "hipSetDevice");
    SG_HIP(hipMemcpyAsync(data, b->ptr + off, size, hipMemcpyDeviceToHost, s->s), "hipMemcpyAsync");
    return finish(s, 1, "buffer_read");
    (void) blocking;
}

scrapgpu_status api_buffer_copy(scrapgpu_stream_t * stream, scrapgpu_buffer_t * dst, uint64_t doff, scrapgpu_buffer_t * src, uint64_t soff, size_t size, int blocking) {
    Stream * s = stream_of(stream);
    Buffer * bd = buf_of(dst);
    Buffer * bs = buf_of(src);
    scrapgpu_status st = check_range(s, bd, doff, size);
    if (st == SCRAPGPU_STATUS_OK) st = check_range(s, bs, soff, size);
    if (st != SCRAPGPU_STATUS_OK || size == 0) return st;
    SG_HIP(use(s->dev), "hipSetDevice");
    SG_HIP(hipMemcpyAsync(bd->ptr + doff, bs->ptr + soff, size, hipMemcpyDeviceToDevice, s->s), "hipMemcpyAsync");
    return finish(s, blocking, "buffer_copy");
}

scrapgpu_status api_buffer_fill(scrapgpu_stream_t * stream, scrapgpu_buffer_t * buffer, uint64_t off, size_t size, uint8_t byte, int blocking) {
    Stream * s = stream_of(stream);
    Buffer * b = buf_of(buffer);
    scrapgpu_status st = check_range(s, b, off, size);
    if (st != SCRAPGPU_STATUS_OK || size == 0) return st;
    SG_HIP(use(s->dev), "hipSetDevice");
    SG_HIP(hipMemsetD8Async(reinterpret_cast<hipDeviceptr_t>(b->ptr + off), byte, size, s->s), "hipMemsetD8Async");
    return finish(s, blocking, "buffer_fill");
}

// ---- streams ----------------------------------------------------------------------------------------

scrapgpu_status api_stream_create(scrapgpu_device_t * device, scrapgpu_stream_t ** out) {
    Device * d = dev_of(device);
    if (d == nullptr) return invalid("not a hip device");
    SG_HIP(use(d), "hipSetDevice");
    hipStream_t hs;
    SG_HIP(hipStreamCreateWithFlags(&hs, hipStreamNonBlocking), "hipStreamCreate");
    // the chunked matvec's arrival counts: zeroed here, once (every launch leaves them at zero)
    uint32_t * arrive = nullptr;
    hipError_t e = hipMalloc(reinterpret_cast<void **>(&arrive), (size_t) sgk::kArriveMax * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(arrive, 0, (size_t) sgk::kArriveMax * sizeof(uint32_t));
    if (e != hipSuccess) {
        if (arrive) hipFree(arrive);
        hipStreamDestroy(hs);
        return hip_fail(e, "hipMalloc / hipMemset (stream arrival counts)");
    }
    Stream * s = new Stream;
    s->hdr.backend = &kVtable;
    s->dev = d;
    s->s = hs;
    s->arrive = arrive;
    s->scratch_gen = g_scratch_gen.fetch_add(1);
    *out = reinterpret_cast<scrapgpu_stream_t *>(s);
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status api_stream_free(scrapgpu_stream_t * stream) {
    Stream * s = stream_of(stream);
    if (s == nullptr) return invalid("not a hip stream");
    use(s->dev);
    hipStreamSynchronize(s->s);
    if (s->scratch) hipFree(s->scratch);
    if (s->arrive) hipFree(s->arrive);
    hipStreamDestroy(s->s);
    delete s;
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status api_stream_sync(scrapgpu_stream_t * stream) {
    Stream * s = stream_of(stream);
    if (s == nullptr) return invalid("not a hip stream");
    SG_HIP(use(s->dev), "hipSetDevice");
    SG_HIP(hipStreamSynchronize(s->s), "kernel execution failed (reported at stream_sync)");
    return SCRAPGPU_STATUS_OK;
}

} // namespace

// The scratch of scrapgpu_hip_op_execute_static: a file-scope device array, so that entry point
// allocates nothing. Each GPU holds its own copy (its address comes from hipGetSymbolAddress at
// registration, per device; the host-side name is not a device address and is never passed to a
// kernel). Every static call on one GPU shares it.
constexpr size_t kStaticScratchBytes = (size_t) 32 << 20;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
// ... and its arrival counts of the chunked decode matvec: zero at load, left at zero by every
// launch (the stream's own counts play this part in scrapgpu_op_execute)
static __device__ __align__(256) uint32_t arrive_counts[sgk::kArriveMax];

namespace {

// stream scratch: grown on demand; the stream is drained before the old block is released
scrapgpu_status ensure_scratch(Stream * s, size_t bytes) {
    if (bytes <= s->scratch_size) return SCRAPGPU_STATUS_OK;
    SG_HIP(hipStreamSynchronize(s->s), "hipStreamSynchronize");
    if (s->scratch) hipFree(s->scratch);
    s->scratch = nullptr;
    s->scratch_size = 0;
    const size_t n = std::max(bytes, (size_t) 16 << 20);
    SG_HIP(hipMalloc(reinterpret_cast<void **>(&s->scratch), n), "hipMalloc (stream scratch)");
    s->scratch_size = n;
    s->scratch_gen = g_scratch_gen.fetch_add(1);
    return SCRAPGPU_STATUS_OK;
}

// `bytes` of scratch for the op being enqueued: the device's static array inside
// scrapgpu_hip_op_execute_static (refused past its size, nothing allocated), else the stream's
// scratch, grown on demand
scrapgpu_status scratch_for(Stream * s, size_t bytes, uint8_t ** out) {
    if (t_static_scratch != nullptr) {
        if (bytes > kStaticScratchBytes) {
            return set_err(SCRAPGPU_STATUS_UNSUPPORTED, "the op needs " + std::to_string(bytes) + " bytes of scratch; the static scratch of "
                                                        "scrapgpu_hip_op_execute_static holds " + std::to_string(kStaticScratchBytes) +
                                                        " (run it with scrapgpu_op_execute)");
        }
        *out = t_static_scratch;
        return SCRAPGPU_STATUS_OK;
    }
    const scrapgpu_status st = ensure_scratch(s, bytes);
    *out = s->scratch;
    return st;
}

scrapgpu_device_t * api_stream_device(scrapgpu_stream_t * stream) {
    Stream * s = stream_of(stream);
    return s ? reinterpret_cast<scrapgpu_device_t *>(s->dev) : nullptr;
}

// ---- tensor transfers with R32 packing in HBM ------------------------------------------------------

constexpr size_t kStagingBytes = (size_t) 64 << 20;

scrapgpu_status ensure_staging(Device * d) {
    if (d->staging) return SCRAPGPU_STATUS_OK;
    SG_HIP(hipMalloc(reinterpret_cast<void **>(&d->staging), kStagingBytes), "hipMalloc (staging)");
    d->staging_size = kStagingBytes;
    return SCRAPGPU_STATUS_OK;
}

// Copies the first `size` natural bytes of an R32 tensor between the host and the device, one chunk
// of whole 32-row groups of a slice at a time through the device staging buffer. A chunk that the
// host range only partly covers is unpacked first so the bytes beyond `size` are preserved.
scrapgpu_status r32_transfer(Stream * s, const scrapgpu_tensor_desc & t, uint8_t * dev_base, uint8_t * host, size_t size, bool up) {
    Device * d = s->dev;
    const int64_t K = t.ne[0], M = sg::dim1(t.ne[1]);
    const int64_t slices = sg::dim1(t.ne[2]) * sg::dim1(t.ne[3]);
    const sg::R32Geom g = sg::r32_geometry(t.dtype, K, M);
    if (g.rowb == 0) return invalid("R32 tensor has no whole block per row");
    const size_t slice_bytes = (size_t) M * g.rowb;
    std::lock_guard<std::mutex> lock(d->mu);
    scrapgpu_status st = ensure_staging(d);
    if (st != SCRAPGPU_STATUS_OK) return st;
    const int64_t chunk_rows = std::max<int64_t>(32, (int64_t) (d->staging_size / g.rowb) / 32 * 32);
    for (int64_t sl = 0; sl < slices; ++sl) {
        const size_t slice_lo = (size_t) sl * slice_bytes;
        if (slice_lo >= size) break;
        uint8_t * rep = dev_base + slice_lo; // slices are stored back to back, like the natural layout
        for (int64_t rA = 0; rA < M; rA += std::min<int64_t>(chunk_rows, 32 * 65535)) {
            const int64_t rB = std::min<int64_t>(M, rA + std::min<int64_t>(chunk_rows, 32 * 65535));
            const size_t nat_lo = slice_lo + (size_t) rA * g.rowb;
            if (nat_lo >= size) break;
            const size_t nat_len = (size_t) (rB - rA) * g.rowb;
            const size_t have = std::min(nat_len, size - nat_lo);
            if (up) {
                if (have < nat_len) {
                    SG_HIP(sgk::launch_r32_move(t.dtype, K, M, rA, rB - rA, d->staging, rep, false, s->s), "R32 unpack");
                }
                SG_HIP(hipMemcpyAsync(d->staging, host + nat_lo, have, hipMemcpyHostToDevice, s->s), "hipMemcpyAsync");
                SG_HIP(sgk::launch_r32_move(t.dtype, K, M, rA, rB - rA, d->staging, rep, true, s->s), "R32 pack");
            } else {
                SG_HIP(sgk::launch_r32_move(t.dtype, K, M, rA, rB - rA, d->staging, rep, false, s->s), "R32 unpack");
                SG_HIP(hipMemcpyAsync(host + nat_lo, d->staging, have, hipMemcpyDeviceToHost, s->s), "hipMemcpyAsync");
            }
            // the staging buffer is reused by the next chunk (same stream: ordered)
        }
    }
    SG_HIP(hipStreamSynchronize(s->s), "R32 transfer");
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status tensor_transfer(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * raw, uint8_t * host, size_t size, bool up) {
    Stream * s = stream_of(stream);
    if (s == nullptr) return invalid("not a hip stream");
    if (raw->struct_size < offsetof(scrapgpu_tensor_desc, offset) + sizeof(raw->offset)) return invalid("the tensor desc is shorter than its required fields");
    const scrapgpu_tensor_desc t = load_desc(*raw);
    Buffer * b = buf_of(t.buffer);
    if (b == nullptr) return invalid("tensor desc has no hip buffer");
    if (b->dev != s->dev) return invalid("the tensor's buffer lives on another device than the stream");
    if (t.offset > b->size || size > b->size - t.offset) return invalid("the transfer reaches past the end of the buffer");
    if (size > sg::nbytes(t)) return invalid("the transfer is larger than the tensor");
    if (size == 0) return SCRAPGPU_STATUS_OK;
    SG_HIP(use(s->dev), "hipSetDevice");
    if (t.layout == SCRAPGPU_LAYOUT_R32) {
        if (!sg::r32_eligible(t)) return unsupported("R32 needs a Q4_0/Q8_0/Q4_K/Q6_K tensor with contiguous rows, whole blocks per row and slice strides that are multiples of 16 bytes");
        return r32_transfer(s, t, b->ptr + t.offset, host, size, up);
    }
    if (!sg::contiguous_ggml(t)) return unsupported("only contiguous tensors transfer through tensor_upload/download; strided data goes through buffer_write/buffer_read");
    if (up) {
        SG_HIP(hipMemcpyAsync(b->ptr + t.offset, host, size, hipMemcpyHostToDevice, s->s), "hipMemcpyAsync");
    } else {
        SG_HIP(hipMemcpyAsync(host, b->ptr + t.offset, size, hipMemcpyDeviceToHost, s->s), "hipMemcpyAsync");
    }
    SG_HIP(hipStreamSynchronize(s->s), "tensor transfer");
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status api_tensor_upload(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * desc, const void * host, size_t size) {
    return tensor_transfer(stream, desc, static_cast<uint8_t *>(const_cast<void *>(host)), size, true);
}

scrapgpu_status api_tensor_download(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * desc, void * host, size_t size) {
    return tensor_transfer(stream, desc, static_cast<uint8_t *>(host), size, false);
}

// ---- MUL_MAT ------------------------------------------------------------------------------------------

// the support rule of one product W x -> y; fills `a` (pointers left null) when supported
scrapgpu_status mul_mat_rule(const scrapgpu_tensor_desc & w, const scrapgpu_tensor_desc & x, const scrapgpu_tensor_desc & y, int allow_broadcast,
                             sgk::MatArgs * a, const char ** reason) {
    const bool fw = w.dtype == SCRAPGPU_DTYPE_F32 || w.dtype == SCRAPGPU_DTYPE_F16 || w.dtype == SCRAPGPU_DTYPE_BF16;
    if (!sg::is_quant(w.dtype) && !fw) {
        return unsupported("the hip backend implements MUL_MAT for Q4_0 / Q8_0 / Q4_K / Q6_K, F32, F16 and BF16 weights", reason);
    }
    if (fw) {
        // float weights (the reference's exec_mul_mat reads them with load_float): natural rows
        if (w.layout != SCRAPGPU_LAYOUT_NATURAL) return unsupported("float weights run from the natural layout", reason);
        if (w.nb[0] != sg::type_size(w.dtype)) return unsupported("MUL_MAT needs contiguous rows of src0 (nb0 == element size)", reason);
        if (sg::dim1(w.ne[0]) % 8 != 0) return unsupported("float weights: the hip kernels read rows in runs of 8 elements, so K must be a multiple of 8", reason);
        if (w.nb[1] % 16 != 0 || w.nb[2] % 16 != 0 || w.nb[3] % 16 != 0 || w.offset % 16 != 0) {
            return unsupported("float weights: rows and slices must start on 16-byte boundaries", reason);
        }
    } else {
        if (w.layout != SCRAPGPU_LAYOUT_R32) {
            return unsupported("quantized weights run from the R32 layout only: upload them with layout R32 (the upload repacks natural blocks)", reason);
        }
        if (!sg::r32_eligible(w)) return unsupported("src0 is not R32-eligible (contiguous, whole blocks per row, 16-byte slice strides)", reason);
    }
    if (x.dtype != SCRAPGPU_DTYPE_F32 || y.dtype != SCRAPGPU_DTYPE_F32 || x.layout != SCRAPGPU_LAYOUT_NATURAL || y.layout != SCRAPGPU_LAYOUT_NATURAL) {
        return unsupported("MUL_MAT expects an F32 natural-layout src1 and destination", reason);
    }
    if (x.nb[0] != 4 || y.nb[0] != 4) return unsupported("MUL_MAT: src1 and dst rows must be packed floats (nb0 == 4)", reason);
    for (int i = 1; i < 4; ++i) {
        if (x.nb[i] % 4 != 0 || y.nb[i] % 4 != 0) return unsupported("src1 / dst strides must be multiples of 4 bytes", reason);
    }
    if ((x.offset % 4) != 0 || (y.offset % 4) != 0) return unsupported("src1 / dst offsets must be multiples of 4 bytes", reason);
    const int64_t K = sg::dim1(w.ne[0]), M = sg::dim1(w.ne[1]);
    if (sg::dim1(x.ne[0]) != K) {
        if (reason) *reason = "MUL_MAT: src0 and src1 disagree on K (ne0)";
        return invalid("MUL_MAT: src0 and src1 disagree on K (ne0)");
    }
    const int64_t w2 = sg::dim1(w.ne[2]), w3 = sg::dim1(w.ne[3]);
    const int64_t x2 = sg::dim1(x.ne[2]), x3 = sg::dim1(x.ne[3]);
    if (x2 % w2 != 0 || x3 % w3 != 0) {
        if (reason) *reason = "MUL_MAT: src1 slice counts (ne2, ne3) must be whole multiples of src0's";
        return invalid("MUL_MAT: src1 slice counts (ne2, ne3) must be whole multiples of src0's");
    }
    if (!allow_broadcast && (x2 != w2 || x3 != w3)) return unsupported("MUL_MAT: src0 has fewer slices than src1 and allow_broadcast is 0 (no broadcast)", reason);
    if (sg::dim1(y.ne[0]) != M || sg::dim1(y.ne[1]) != sg::dim1(x.ne[1]) || sg::dim1(y.ne[2]) != x2 || sg::dim1(y.ne[3]) != x3) {
        if (reason) *reason = "MUL_MAT: dst shape is not [src0 ne1, src1 ne1, src1 ne2, src1 ne3]";
        return invalid("MUL_MAT: dst shape is not [src0 ne1, src1 ne1, src1 ne2, src1 ne3]");
    }
    if (x2 * x3 > 65535) return unsupported("MUL_MAT: more than 65535 slices", reason);
    // the kernels address one slice of weights, and one slice of x in f16, with 32-bit offsets
    if (sg::sat_mul(fw ? std::max<uint64_t>(w.nb[1], sg::row_size(w.dtype, K)) : sg::row_size(w.dtype, K), (uint64_t) M) >= ((uint64_t) 1 << 32)) {
        return unsupported("MUL_MAT: one slice of src0 must be smaller than 4 GiB", reason);
    }
    if (sg::sat_mul((uint64_t) K, (uint64_t) sg::dim1(x.ne[1])) >= ((uint64_t) 1 << 31)) {
        return unsupported("MUL_MAT: one slice of src1 must hold fewer than 2^31 elements", reason);
    }
    if (a) {
        a->dtype = w.dtype;
        a->M = M;
        a->K = K;
        a->nb = fw ? (int64_t) w.nb[1] : K / (int64_t) sg::block_size(w.dtype); // (float weights: the row stride in bytes)
        a->w_s2 = w.nb[2];
        a->w_s3 = w.nb[3];
        a->x_s1 = (int64_t) (x.nb[1] / 4);
        a->x_s2 = (int64_t) (x.nb[2] / 4);
        a->x_s3 = (int64_t) (x.nb[3] / 4);
        a->y_s1 = (int64_t) (y.nb[1] / 4);
        a->y_s2 = (int64_t) (y.nb[2] / 4);
        a->y_s3 = (int64_t) (y.nb[3] / 4);
        a->N = sg::dim1(x.ne[1]);
        a->ne12 = x2;
        a->ne13 = x3;
        a->r2 = x2 / w2;
        a->r3 = x3 / w3;
    }
    return SCRAPGPU_STATUS_OK;
}

// the support rule of MUL_MAT_ID (reference ops.cpp:986-1024, opencl11/ops_moe.cpp): experts
// w [K, M, E] quantized R32, x F32 [K, 1 or n_used, T], ids I32 [n_used, T], dst F32 [M, n_used, T].
// Fills `a` / `id` (pointers left null) when supported. One (slot, token) pair per matvec slice.
scrapgpu_status mul_mat_id_rule(const scrapgpu_tensor_desc & w, const scrapgpu_tensor_desc & x, const scrapgpu_tensor_desc & ids,
                                const scrapgpu_tensor_desc & y, sgk::MatArgs * a, sgk::IdArgs * id, const char ** reason) {
    const bool fw = w.dtype == SCRAPGPU_DTYPE_F32 || w.dtype == SCRAPGPU_DTYPE_F16;
    if (!sg::is_quant(w.dtype) && !fw) return unsupported("the hip backend implements MUL_MAT_ID for Q4_0 / Q8_0 / Q4_K / Q6_K, F32 and F16 experts", reason);
    if (fw) {
        // (reference ops.cpp:986-1024 reads F32 / F16 experts with load_float): natural rows
        if (w.layout != SCRAPGPU_LAYOUT_NATURAL) return unsupported("float experts run from the natural layout", reason);
        if (w.nb[0] != sg::type_size(w.dtype)) return unsupported("MUL_MAT_ID needs contiguous rows of src0 (nb0 == element size)", reason);
        if (sg::dim1(w.ne[0]) % 8 != 0) return unsupported("float experts: the hip kernels read rows in runs of 8 elements, so K must be a multiple of 8", reason);
        if (w.nb[1] % 16 != 0 || w.nb[2] % 16 != 0 || w.offset % 16 != 0) return unsupported("float experts: rows and experts must start on 16-byte boundaries", reason);
    } else {
        if (w.layout != SCRAPGPU_LAYOUT_R32) {
            return unsupported("quantized experts must use the R32 layout (scrapgpu_tensor_upload packs them on the way)", reason);
        }
        if (!sg::r32_eligible(w)) return unsupported("src0 is not R32-eligible (contiguous, whole blocks per row, 16-byte slice strides)", reason);
    }
    if (x.dtype != SCRAPGPU_DTYPE_F32 || y.dtype != SCRAPGPU_DTYPE_F32 || x.layout != SCRAPGPU_LAYOUT_NATURAL || y.layout != SCRAPGPU_LAYOUT_NATURAL) {
        return unsupported("MUL_MAT_ID expects an F32 natural-layout src1 and destination", reason);
    }
    if (ids.dtype != SCRAPGPU_DTYPE_I32 || ids.layout != SCRAPGPU_LAYOUT_NATURAL) return unsupported("MUL_MAT_ID expects I32 ids", reason);
    if (x.nb[0] != 4 || y.nb[0] != 4 || ids.nb[0] != 4) return unsupported("MUL_MAT_ID needs contiguous rows of src1, ids and dst", reason);
    for (int i = 1; i < 4; ++i) {
        if (x.nb[i] % 4 != 0 || y.nb[i] % 4 != 0 || ids.nb[i] % 4 != 0) return unsupported("src1 / ids / dst strides must be multiples of 4 bytes", reason);
    }
    if (x.offset % 4 != 0 || y.offset % 4 != 0 || ids.offset % 4 != 0) return unsupported("src1 / ids / dst offsets must be multiples of 4 bytes", reason);
    const int64_t K = sg::dim1(w.ne[0]), M = sg::dim1(w.ne[1]), E = sg::dim1(w.ne[2]);
    const int64_t nu = sg::dim1(ids.ne[0]), T = sg::dim1(ids.ne[1]);
    if (sg::dim1(w.ne[3]) != 1 || sg::dim1(x.ne[3]) != 1 || sg::dim1(ids.ne[2]) != 1 || sg::dim1(ids.ne[3]) != 1 || sg::dim1(x.ne[0]) != K ||
        (sg::dim1(x.ne[1]) != 1 && sg::dim1(x.ne[1]) != nu) || sg::dim1(x.ne[2]) != T || sg::dim1(y.ne[0]) != M || sg::dim1(y.ne[1]) != nu ||
        sg::dim1(y.ne[2]) != T || sg::dim1(y.ne[3]) != 1) {
        if (reason) *reason = "MUL_MAT_ID needs [K,M,E] src0, [K,n_used|1,n_tokens] src1, I32 [n_used,n_tokens] ids and [M,n_used,n_tokens] dst";
        return invalid("MUL_MAT_ID: src1, ids and dst shapes are inconsistent with src0 and n_used");
    }
    if (nu * T > 65535) return unsupported("MUL_MAT_ID: more than 65535 (slot, token) pairs", reason);
    if (sg::sat_mul(fw ? std::max<uint64_t>(w.nb[1], sg::row_size(w.dtype, K)) : sg::row_size(w.dtype, K), (uint64_t) M) >= ((uint64_t) 1 << 32)) {
        return unsupported("MUL_MAT_ID: one expert must be smaller than 4 GiB", reason);
    }
    if (a) {
        std::memset(a, 0, sizeof(*a));
        a->dtype = w.dtype;
        a->M = M;
        a->K = K;
        a->nb = fw ? (int64_t) w.nb[1] : K / (int64_t) sg::block_size(w.dtype); // (float experts: the row stride in bytes)
        a->w_s2 = w.nb[2];
        a->x_s1 = (int64_t) (x.nb[1] / 4);
        a->x_s2 = (int64_t) (x.nb[2] / 4);
        a->y_s1 = (int64_t) (y.nb[1] / 4);
        a->y_s2 = (int64_t) (y.nb[2] / 4);
        a->N = 1;
        a->ne12 = 1;
        a->ne13 = 1;
        a->r2 = 1;
        a->r3 = 1;
    }
    if (id) {
        id->ids = nullptr;
        id->s0 = (int64_t) (ids.nb[0] / 4);
        id->s1 = (int64_t) (ids.nb[1] / 4);
        id->n_used = nu;
        id->n_tok = T;
        id->n_exp = E;
        id->x_shared = sg::dim1(x.ne[1]) == 1 ? 1 : 0;
    }
    return SCRAPGPU_STATUS_OK;
}

// the support rule of GET_ROWS (reference ops.cpp:690-721, opencl11/ops_support.cpp:82-88) on
// R32 weights: src0 [K, R, S2, S3] quantized R32, ids I32 [n0, n1 <= S2, n2 <= S3], dst F32
// [K, n0, n1, n2]. Fills `g` (pointers left null) when supported.
scrapgpu_status get_rows_rule(const scrapgpu_tensor_desc & w, const scrapgpu_tensor_desc & ids, const scrapgpu_tensor_desc & y,
                              sgk::GetRowsLaunch * g, const char ** reason) {
    const bool fw = w.dtype == SCRAPGPU_DTYPE_F32 || w.dtype == SCRAPGPU_DTYPE_F16;
    if (!sg::is_quant(w.dtype) && !fw) return unsupported("the hip backend implements GET_ROWS for Q4_0 / Q8_0 / Q4_K / Q6_K, F32 and F16 rows", reason);
    if (fw) {
        // (reference ops.cpp:690-721 reads F32 / F16 rows with load_float)
        if (w.layout != SCRAPGPU_LAYOUT_NATURAL) return unsupported("F32 / F16 GET_ROWS sources use the natural layout", reason);
        if (w.nb[0] != sg::type_size(w.dtype)) return unsupported("GET_ROWS needs contiguous rows (nb0 == element size)", reason);
        for (int i = 1; i < 4; ++i) {
            if (w.nb[i] % w.nb[0] != 0) return unsupported("GET_ROWS: src0 strides must be whole elements", reason);
        }
        if (w.offset % w.nb[0] != 0) return unsupported("GET_ROWS: the src0 offset must be a whole element", reason);
    } else {
        if (w.layout != SCRAPGPU_LAYOUT_R32) {
            return unsupported("quantized GET_ROWS sources must use the R32 layout (scrapgpu_tensor_upload packs them on the way)", reason);
        }
        if (!sg::r32_eligible(w)) return unsupported("src0 is not R32-eligible (contiguous, whole blocks per row, 16-byte slice strides)", reason);
    }
    if (ids.dtype != SCRAPGPU_DTYPE_I32 || ids.layout != SCRAPGPU_LAYOUT_NATURAL || y.dtype != SCRAPGPU_DTYPE_F32 || y.layout != SCRAPGPU_LAYOUT_NATURAL) {
        return unsupported("GET_ROWS expects I32 indices and an F32 natural-layout destination", reason);
    }
    if (ids.nb[0] != 4 || y.nb[0] != 4) return unsupported("GET_ROWS needs contiguous rows of ids and dst", reason);
    for (int i = 1; i < 4; ++i) {
        if (ids.nb[i] % 4 != 0 || y.nb[i] % 4 != 0) return unsupported("ids / dst strides must be multiples of 4 bytes", reason);
    }
    if (ids.offset % 4 != 0 || y.offset % 4 != 0) return unsupported("ids / dst offsets must be multiples of 4 bytes", reason);
    const int64_t K = sg::dim1(w.ne[0]);
    if (sg::dim1(ids.ne[3]) != 1 || sg::dim1(ids.ne[1]) > sg::dim1(w.ne[2]) || sg::dim1(ids.ne[2]) > sg::dim1(w.ne[3]) || sg::dim1(y.ne[0]) != K ||
        sg::dim1(y.ne[1]) != sg::dim1(ids.ne[0]) || sg::dim1(y.ne[2]) != sg::dim1(ids.ne[1]) || sg::dim1(y.ne[3]) != sg::dim1(ids.ne[2])) {
        if (reason) *reason = "GET_ROWS: dst shape is not [src0 ne0, ids ne0, ids ne1, ids ne2]";
        return invalid("GET_ROWS: dst shape is not [src0 ne0, ids ne0, ids ne1, ids ne2]");
    }
    if (g) {
        std::memset(g, 0, sizeof(*g));
        g->dtype = w.dtype;
        g->w_s1 = w.nb[1];
        g->w_s2 = w.nb[2];
        g->w_s3 = w.nb[3];
        g->i_s0 = (int64_t) (ids.nb[0] / 4);
        g->i_s1 = (int64_t) (ids.nb[1] / 4);
        g->i_s2 = (int64_t) (ids.nb[2] / 4);
        g->y_s1 = (int64_t) (y.nb[1] / 4);
        g->y_s2 = (int64_t) (y.nb[2] / 4);
        g->y_s3 = (int64_t) (y.nb[3] / 4);
        g->K = K;
        g->M = sg::dim1(w.ne[1]);
        g->n0 = sg::dim1(ids.ne[0]);
        g->n1 = sg::dim1(ids.ne[1]);
        g->n2 = sg::dim1(ids.ne[2]);
    }
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status api_supports(Device * d, const scrapgpu_op_desc * desc, const char ** reason) {
    (void) d;
    const scrapgpu_status v = scrapgpu_op_desc_validate(desc);
    if (v != SCRAPGPU_STATUS_OK) {
        if (reason) *reason = scrapgpu_last_error();
        return v;
    }
    switch (desc->op) {
        case SCRAPGPU_OP_MUL_MAT: {
            const auto * p = static_cast<const scrapgpu_mul_mat_params *>(desc->params);
            const int bc = p->struct_size >= offsetof(scrapgpu_mul_mat_params, allow_broadcast) + sizeof(int) ? p->allow_broadcast : 0;
            return mul_mat_rule(desc->inputs[0], desc->inputs[1], desc->outputs[0], bc, nullptr, reason);
        }
        case SCRAPGPU_OP_MUL_MAT_MULTI: {
            const size_t n = desc->output_count;
            for (size_t i = 0; i < n; ++i) {
                const scrapgpu_status st = mul_mat_rule(desc->inputs[i], desc->inputs[n], desc->outputs[i], 0, nullptr, reason);
                if (st != SCRAPGPU_STATUS_OK) return st;
            }
            return SCRAPGPU_STATUS_OK;
        }
        case SCRAPGPU_OP_MUL_MAT_ID:
            return mul_mat_id_rule(desc->inputs[0], desc->inputs[1], desc->inputs[2], desc->outputs[0], nullptr, nullptr, reason);
        case SCRAPGPU_OP_GET_ROWS:
            return get_rows_rule(desc->inputs[0], desc->inputs[1], desc->outputs[0], nullptr, reason);
        default:
            return unsupported("the hip backend implements the quantized MUL_MAT family only", reason);
    }
}

scrapgpu_status api_op_supported(scrapgpu_device_t * device, const scrapgpu_op_desc * desc, const char ** reason) {
    Device * d = dev_of(device);
    if (d == nullptr) {
        if (reason) *reason = "not a hip device";
        return invalid("not a hip device");
    }
    return api_supports(d, desc, reason);
}

double weight_bytes(const sgk::MatArgs & a) {
    if (sgk::is_float_weight(a.dtype)) {
        return (double) a.M * (double) a.K * (a.dtype == sgk::F32 ? 4.0 : 2.0) * (double) ((a.ne12 / a.r2) * (a.ne13 / a.r3));
    }
    const int64_t bs = a.dtype == sgk::Q4_K || a.dtype == sgk::Q6_K ? 256 : 32;
    const double ts = a.dtype == sgk::Q4_0 ? 18 : a.dtype == sgk::Q8_0 ? 34 : a.dtype == sgk::Q4_K ? 144 : 210;
    return (double) a.M * (double) (a.K / bs) * ts * (double) ((a.ne12 / a.r2) * (a.ne13 / a.r3));
}

// enqueues 1..3 products on the stream (pointers resolved). Products that share x with one dtype,
// K and N <= 8 run as one fused matvec launch; anything else as one launch per product.
// MUL_MAT_ID takes the grouped MFMA path for more than 8 tokens once the experts average 4 pairs
// or more (the matvec path reads an expert once per pair; with fewer pairs per expert it is as
// fast), within the routing kernel's limits
bool mul_mat_id_grouped(const sgk::MatArgs & a, const sgk::IdArgs & id) {
    const int64_t rows = (id.x_shared ? 1 : id.n_used) * id.n_tok;
    return !sgk::is_float_weight(a.dtype) && id.n_tok > 8 && id.n_used * id.n_tok >= 4 * id.n_exp && id.n_exp <= 1024 && rows * a.K < ((int64_t) 1 << 31);
}

// the largest column count that takes the decode matvec (above it: the f16 MFMA GEMM). 8 keeps
// batch decode on the matvec's integer path (NMSE ~1e-10; the GEMM's f16 operands give ~1e-7);
// by speed the GEMM wins from 8 columns on the MLP shapes and from 4 (Q6_K, K = 12288)
int64_t matvec_max_n(const sgk::MatArgs & a) {
    static const int env = [] {
        const char * v = std::getenv("SCRAPGPU_HIP_MV_MAXN");
        return v != nullptr && *v ? std::atoi(v) : 0;
    }();
    (void) a;
    return env >= 1 && env <= 8 ? env : 8;
}

scrapgpu_status run_products(Stream * s, const sgk::MatArgs * mats, int n) {
    const int cus = (int) s->dev->cus;
    const int64_t mv_n = matvec_max_n(mats[0]);
    bool fuse = n > 1 && mats[0].N <= mv_n;
    for (int j = 1; j < n && fuse; ++j) {
        fuse = mats[j].dtype == mats[0].dtype && mats[j].K == mats[0].K && mats[j].x == mats[0].x &&
               mats[j].ne12 * mats[j].ne13 == 1 && mats[0].ne12 * mats[0].ne13 == 1;
    }
    // prefill weights of one dtype reading the same x (one slice each): one GEMM launch over all
    bool fuse_mm = n > 1 && mats[0].N > mv_n && mats[0].ne12 * mats[0].ne13 == 1;
    for (int j = 1; j < n && fuse_mm; ++j) {
        fuse_mm = mats[j].dtype == mats[0].dtype && sgk::matmul_reads_same_x(mats[j], mats[0]) && mats[j].ne12 * mats[j].ne13 == 1;
    }
    if (fuse_mm) {
        sgk::MatArgs all = mats[0];
        double bytes = 0, flops = 0;
        for (int j = 0; j < n; ++j) {
            if (j > 0) all.M += mats[j].M;
            bytes += weight_bytes(mats[j]);
            flops += 2.0 * (double) mats[j].M * (double) mats[j].K * (double) mats[j].N;
        }
        uint8_t * scr = nullptr;
        const bool lean = t_static_scratch != nullptr;
        const scrapgpu_status st = scratch_for(s, sgk::matmul_scratch_bytes(all, cus, lean), &scr);
        if (st != SCRAPGPU_STATUS_OK) return st;
        ProfScope prof(s->s);
        const char * name = nullptr;
        SG_HIP(sgk::launch_matmul_mfma(mats, n, scr, cus, s->s, &name, false, lean), "matmul (MULTI) launch");
        prof.done(name, bytes, flops);
        return SCRAPGPU_STATUS_OK;
    }
    const int groups = fuse ? 1 : n;
    if (!fuse && n > 1 && mats[0].N > mv_n) {
        // prefill products of one MUL_MAT_MULTI: scratch for the largest first, so that products
        // reading the same x share one x pre-pass (the scratch stays in place between them)
        size_t need = 0;
        for (int j = 0; j < n; ++j) need = std::max(need, sgk::matmul_scratch_bytes(mats[j], cus, t_static_scratch != nullptr));
        uint8_t * scr = nullptr;
        const scrapgpu_status st = scratch_for(s, need, &scr);
        if (st != SCRAPGPU_STATUS_OK) return st;
    }
    for (int gi = 0; gi < groups; ++gi) {
        const sgk::MatArgs * m = fuse ? mats : mats + gi;
        const int cnt = fuse ? n : 1;
        double bytes = 0, flops = 0;
        for (int j = 0; j < cnt; ++j) {
            bytes += weight_bytes(m[j]);
            flops += 2.0 * (double) m[j].M * (double) m[j].K * (double) m[j].N * (double) (m[j].ne12 * m[j].ne13);
        }
        if (m[0].N <= mv_n) {
            uint8_t * scr = nullptr;
            if (const size_t need = sgk::matvec_scratch_bytes(m, cnt)) {
                const scrapgpu_status st = scratch_for(s, need, &scr);
                if (st != SCRAPGPU_STATUS_OK) return st;
            }
            ProfScope prof(s->s);
            const char * name = nullptr;
            uint64_t grid = 0;
            uint32_t * arrive = t_static_scratch != nullptr ? t_static_arrive : s->arrive;
            SG_HIP(sgk::launch_matvec(m, cnt, cus, s->s, &name, &grid, nullptr, scr, arrive), "matvec launch");
            prof.done(name, bytes, flops);
        } else {
            uint8_t * scr = nullptr;
            const bool lean = t_static_scratch != nullptr;
            const scrapgpu_status st = scratch_for(s, sgk::matmul_scratch_bytes(m[0], cus, lean), &scr);
            if (st != SCRAPGPU_STATUS_OK) return st;
            ProfScope prof(s->s);
            const char * name = nullptr;
            const bool x_ready = !fuse && gi > 0 && mats[gi - 1].N > mv_n && sgk::matmul_same_x(mats[gi - 1], m[0], cus, lean);
            SG_HIP(sgk::launch_matmul_mfma(m, 1, scr, cus, s->s, &name, x_ready, lean), "matmul launch");
            prof.done(name, bytes, flops);
        }
    }
    return SCRAPGPU_STATUS_OK;
}

// the resolved arguments of one product W x -> y
scrapgpu_status product_args(Stream * s, const scrapgpu_tensor_desc & w, const scrapgpu_tensor_desc & x, const scrapgpu_tensor_desc & y, int bc,
                             sgk::MatArgs * a) {
    std::memset(a, 0, sizeof(*a));
    scrapgpu_status st = mul_mat_rule(w, x, y, bc, a, nullptr);
    if (st != SCRAPGPU_STATUS_OK) return st;
    uint8_t *pw, *px, *py;
    if ((st = resolve(s->dev, w, &pw, "src0")) != SCRAPGPU_STATUS_OK) return st;
    if ((st = resolve(s->dev, x, &px, "src1")) != SCRAPGPU_STATUS_OK) return st;
    if ((st = resolve(s->dev, y, &py, "dst")) != SCRAPGPU_STATUS_OK) return st;
    a->w = pw;
    a->x = reinterpret_cast<const float *>(px);
    a->y = reinterpret_cast<float *>(py);
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status exec_desc(Stream * s, const scrapgpu_op_desc * desc) {
    const char * reason = nullptr;
    scrapgpu_status st = api_supports(s->dev, desc, &reason);
    if (st != SCRAPGPU_STATUS_OK) return st;
    SG_HIP(use(s->dev), "hipSetDevice");
    sgk::MatArgs mats[3];
    if (desc->op == SCRAPGPU_OP_GET_ROWS) {
        sgk::GetRowsLaunch g;
        st = get_rows_rule(desc->inputs[0], desc->inputs[1], desc->outputs[0], &g, nullptr);
        if (st != SCRAPGPU_STATUS_OK) return st;
        uint8_t *pw, *pi, *py;
        if ((st = resolve(s->dev, desc->inputs[0], &pw, "src0")) != SCRAPGPU_STATUS_OK) return st;
        if ((st = resolve(s->dev, desc->inputs[1], &pi, "ids")) != SCRAPGPU_STATUS_OK) return st;
        if ((st = resolve(s->dev, desc->outputs[0], &py, "dst")) != SCRAPGPU_STATUS_OK) return st;
        g.w = pw;
        g.ids = reinterpret_cast<const int32_t *>(pi);
        g.y = reinterpret_cast<float *>(py);
        const double rows = (double) (g.n0 * g.n1 * g.n2);
        ProfScope prof(s->s);
        SG_HIP(sgk::launch_get_rows(g, s->s), "get_rows launch");
        prof.done("get_rows", rows * (double) sg::row_size(desc->inputs[0].dtype, g.K), 0.0);
        return SCRAPGPU_STATUS_OK;
    }
    if (desc->op == SCRAPGPU_OP_MUL_MAT_ID) {
        sgk::IdArgs id;
        st = mul_mat_id_rule(desc->inputs[0], desc->inputs[1], desc->inputs[2], desc->outputs[0], &mats[0], &id, nullptr);
        if (st != SCRAPGPU_STATUS_OK) return st;
        uint8_t *pw, *px, *pi, *py;
        if ((st = resolve(s->dev, desc->inputs[0], &pw, "src0")) != SCRAPGPU_STATUS_OK) return st;
        if ((st = resolve(s->dev, desc->inputs[1], &px, "src1")) != SCRAPGPU_STATUS_OK) return st;
        if ((st = resolve(s->dev, desc->inputs[2], &pi, "ids")) != SCRAPGPU_STATUS_OK) return st;
        if ((st = resolve(s->dev, desc->outputs[0], &py, "dst")) != SCRAPGPU_STATUS_OK) return st;
        mats[0].w = pw;
        mats[0].x = reinterpret_cast<const float *>(px);
        mats[0].y = reinterpret_cast<float *>(py);
        id.ids = reinterpret_cast<const int32_t *>(pi);
        const double pairs = (double) (id.n_used * id.n_tok);
        if (mul_mat_id_grouped(mats[0], id)) {
            // many tokens: pairs grouped by expert on the device, one MFMA GEMM over them
            uint8_t * scr = nullptr;
            st = scratch_for(s, sgk::mul_mat_id_scratch_bytes(mats[0], id), &scr);
            if (st != SCRAPGPU_STATUS_OK) return st;
            ProfScope prof(s->s);
            const char * name = nullptr;
            SG_HIP(sgk::launch_mul_mat_id_mfma(mats[0], id, scr, (int) s->dev->cus, s->s, &name), "grouped MUL_MAT_ID launch");
            prof.done(name, weight_bytes(mats[0]) * (double) id.n_exp, 2.0 * (double) mats[0].M * (double) mats[0].K * pairs);
            return SCRAPGPU_STATUS_OK;
        }
        ProfScope prof(s->s);
        const char * name = nullptr;
        uint64_t grid = 0;
        SG_HIP(sgk::launch_matvec(mats, 1, (int) s->dev->cus, s->s, &name, &grid, &id), "matvec (MUL_MAT_ID) launch");
        prof.done(name, weight_bytes(mats[0]) * pairs, 2.0 * (double) mats[0].M * (double) mats[0].K * pairs);
        return SCRAPGPU_STATUS_OK;
    }
    if (desc->op == SCRAPGPU_OP_MUL_MAT) {
        const auto * p = static_cast<const scrapgpu_mul_mat_params *>(desc->params);
        const int bc = p->struct_size >= offsetof(scrapgpu_mul_mat_params, allow_broadcast) + sizeof(int) ? p->allow_broadcast : 0;
        st = product_args(s, desc->inputs[0], desc->inputs[1], desc->outputs[0], bc, &mats[0]);
        return st != SCRAPGPU_STATUS_OK ? st : run_products(s, mats, 1);
    }
    const size_t n = desc->output_count; // MUL_MAT_MULTI: n weights sharing inputs[n]
    for (size_t i = 0; i < n; ++i) {
        st = product_args(s, desc->inputs[i], desc->inputs[n], desc->outputs[i], 0, &mats[i]);
        if (st != SCRAPGPU_STATUS_OK) return st;
    }
    return run_products(s, mats, (int) n);
}

bool same_tensor(const scrapgpu_tensor_desc & a, const scrapgpu_tensor_desc & b) {
    if (a.buffer != b.buffer || a.offset != b.offset || a.dtype != b.dtype || a.layout != b.layout) return false;
    for (int i = 0; i < 4; ++i) {
        if (a.ne[i] != b.ne[i] || a.nb[i] != b.nb[i]) return false;
    }
    return true;
}

// true when the byte ranges of two tensors share a byte of one buffer
bool overlap(const scrapgpu_tensor_desc & a, const scrapgpu_tensor_desc & b) {
    if (a.buffer == nullptr || a.buffer != b.buffer) return false;
    const uint64_t ea = a.offset + sg::nbytes(a), eb = b.offset + sg::nbytes(b);
    return a.offset < eb && b.offset < ea;
}

// node b may join a fused group (nodes group[0..n)) only when running them as one launch reads
// and writes what running them in order would: b's output overlaps no input or output of the
// group, and no output of the group overlaps an input of b (checked by byte ranges, so that
// tensors that share one buffer at different offsets still fuse)
bool outputs_apart(const PlanNode * group, int n, const PlanNode & b) {
    const scrapgpu_tensor_desc & yb = b.op.outputs[0];
    for (int k = 0; k < n; ++k) {
        const scrapgpu_op_desc & g = group[k].op;
        const scrapgpu_tensor_desc & yk = g.outputs[0];
        if (overlap(yk, yb)) return false;
        for (size_t i = 0; i < g.input_count; ++i)
            if (overlap(g.inputs[i], yb)) return false;
        for (size_t i = 0; i < b.op.input_count; ++i)
            if (overlap(yk, b.op.inputs[i])) return false;
    }
    for (size_t i = 0; i < b.op.input_count; ++i)
        if (overlap(b.op.inputs[i], yb)) return false;
    return true;
}

// consecutive MUL_MAT_ID nodes of a plan that may share one launch: the same x and ids, experts
// of one dtype, K, count and stride, outputs of one layout apart from every tensor of the group
// (outputs_apart), all on the decode path; or, all on the grouped path, one x pre-pass and
// routing (mul_mat_id_same_x), after which each node runs its GEMM
bool id_fusable(const PlanNode * group, int n, const PlanNode & b, int cu_count) {
    const PlanNode & a = group[0];
    if (a.op.op != SCRAPGPU_OP_MUL_MAT_ID || b.op.op != SCRAPGPU_OP_MUL_MAT_ID) return false;
    sgk::MatArgs ma, mb;
    sgk::IdArgs ia, ib;
    if (mul_mat_id_rule(a.op.inputs[0], a.op.inputs[1], a.op.inputs[2], a.op.outputs[0], &ma, &ia, nullptr) != SCRAPGPU_STATUS_OK ||
        mul_mat_id_rule(b.op.inputs[0], b.op.inputs[1], b.op.inputs[2], b.op.outputs[0], &mb, &ib, nullptr) != SCRAPGPU_STATUS_OK) {
        return false;
    }
    if (!same_tensor(a.op.inputs[1], b.op.inputs[1]) || !same_tensor(a.op.inputs[2], b.op.inputs[2])) return false;
    const bool ga = mul_mat_id_grouped(ma, ia), gb = mul_mat_id_grouped(mb, ib);
    if (ga != gb) return false;
    if (ga) {
        // (x and ids are the same tensors: compare the x forms on the same pointers)
        ma.x = mb.x = nullptr;
        if (ma.dtype != mb.dtype || ia.n_exp != ib.n_exp || ia.n_used != ib.n_used || !sgk::mul_mat_id_same_x(ma, mb, ia, cu_count)) return false;
        return outputs_apart(group, n, b);
    }
    if (ma.dtype != mb.dtype || ma.K != mb.K || ma.w_s2 != mb.w_s2 || ia.n_exp != ib.n_exp || ia.n_used != ib.n_used) return false;
    if (ma.y_s1 != mb.y_s1 || ma.y_s2 != mb.y_s2) return false;
    return outputs_apart(group, n, b);
}

// consecutive MUL_MAT nodes of a plan that may run as one MUL_MAT_MULTI: the same x tensor,
// weights of one dtype and K, one slice, no broadcast, outputs apart from every tensor of the
// group (outputs_apart)
bool mm_fusable(const PlanNode * group, int n, const PlanNode & b) {
    const PlanNode & a = group[0];
    if (a.op.op != SCRAPGPU_OP_MUL_MAT || b.op.op != SCRAPGPU_OP_MUL_MAT) return false;
    sgk::MatArgs ma, mb;
    std::memset(&ma, 0, sizeof(ma));
    std::memset(&mb, 0, sizeof(mb));
    if (mul_mat_rule(a.op.inputs[0], a.op.inputs[1], a.op.outputs[0], 0, &ma, nullptr) != SCRAPGPU_STATUS_OK ||
        mul_mat_rule(b.op.inputs[0], b.op.inputs[1], b.op.outputs[0], 0, &mb, nullptr) != SCRAPGPU_STATUS_OK) {
        return false;
    }
    if (!same_tensor(a.op.inputs[1], b.op.inputs[1])) return false;
    if (ma.dtype != mb.dtype || ma.K != mb.K || ma.ne12 * ma.ne13 != 1 || mb.ne12 * mb.ne13 != 1) return false;
    return outputs_apart(group, n, b);
}

// a plan node and the nodes fused into it: MUL_MAT_IDs sharing x and ids (one matvec launch over
// all their experts) or MUL_MATs sharing x (run as one MUL_MAT_MULTI)
scrapgpu_status exec_node(Stream * s, const PlanNode * nodes) {
    if (nodes[0].fuse == 0) return exec_desc(s, &nodes[0].op);
    const int n = nodes[0].fuse + 1;
    if (nodes[0].op.op == SCRAPGPU_OP_MUL_MAT) {
        sgk::MatArgs mats[3];
        for (int k = 0; k < n; ++k) {
            const scrapgpu_op_desc & op = nodes[k].op;
            const scrapgpu_status st = product_args(s, op.inputs[0], op.inputs[1], op.outputs[0], 0, &mats[k]);
            if (st != SCRAPGPU_STATUS_OK) return st;
        }
        return run_products(s, mats, n);
    }
    sgk::MatArgs mats[3];
    sgk::IdArgs id;
    double bytes = 0, flops = 0;
    for (int k = 0; k < n; ++k) {
        const scrapgpu_op_desc & op = nodes[k].op;
        sgk::IdArgs idk;
        scrapgpu_status st = mul_mat_id_rule(op.inputs[0], op.inputs[1], op.inputs[2], op.outputs[0], &mats[k], &idk, nullptr);
        if (st != SCRAPGPU_STATUS_OK) return st;
        uint8_t *pw, *px, *pi, *py;
        if ((st = resolve(s->dev, op.inputs[0], &pw, "src0")) != SCRAPGPU_STATUS_OK) return st;
        if ((st = resolve(s->dev, op.inputs[1], &px, "src1")) != SCRAPGPU_STATUS_OK) return st;
        if ((st = resolve(s->dev, op.inputs[2], &pi, "ids")) != SCRAPGPU_STATUS_OK) return st;
        if ((st = resolve(s->dev, op.outputs[0], &py, "dst")) != SCRAPGPU_STATUS_OK) return st;
        mats[k].w = pw;
        mats[k].x = reinterpret_cast<const float *>(px);
        mats[k].y = reinterpret_cast<float *>(py);
        idk.ids = reinterpret_cast<const int32_t *>(pi);
        if (k == 0) id = idk;
        const double pairs = (double) (idk.n_used * idk.n_tok);
        bytes += weight_bytes(mats[k]) * pairs;
        flops += 2.0 * (double) mats[k].M * (double) mats[k].K * pairs;
    }
    if (mul_mat_id_grouped(mats[0], id)) {
        // one x pre-pass and routing (with the first node's GEMM), then each further node's GEMM
        // on the same scratch
        size_t need = 0;
        for (int k = 0; k < n; ++k) need = std::max(need, sgk::mul_mat_id_scratch_bytes(mats[k], id));
        uint8_t * scr = nullptr;
        const scrapgpu_status st = scratch_for(s, need, &scr);
        if (st != SCRAPGPU_STATUS_OK) return st;
        for (int k = 0; k < n; ++k) {
            ProfScope prof(s->s);
            const char * name = nullptr;
            SG_HIP(sgk::launch_mul_mat_id_mfma(mats[k], id, scr, (int) s->dev->cus, s->s, &name, k > 0), "grouped MUL_MAT_ID launch");
            prof.done(name, weight_bytes(mats[k]) * (double) id.n_exp, 2.0 * (double) mats[k].M * (double) mats[k].K * (double) (id.n_used * id.n_tok));
        }
        return SCRAPGPU_STATUS_OK;
    }
    ProfScope prof(s->s);
    const char * name = nullptr;
    uint64_t grid = 0;
    SG_HIP(sgk::launch_matvec(mats, n, (int) s->dev->cus, s->s, &name, &grid, &id), "matvec (fused MUL_MAT_ID) launch");
    prof.done(name, bytes, flops);
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status api_op_execute(scrapgpu_stream_t * stream, const scrapgpu_op_desc * desc) {
    Stream * s = stream_of(stream);
    if (s == nullptr) return invalid("not a hip stream");
    if (desc == nullptr) return invalid("op desc is null");
    return exec_desc(s, desc);
}

// ---- plans ------------------------------------------------------------------------------------------------

void plan_release(Plan * p) {
    for (Buffer * b : p->buffers) b->plan_refs.fetch_sub(1);
    p->buffers.clear();
}

scrapgpu_status api_plan_build(scrapgpu_device_t * device, const scrapgpu_plan_desc * desc, scrapgpu_plan_t ** out) {
    Device * d = dev_of(device);
    if (d == nullptr) return invalid("not a hip device");
    if (desc->struct_size < offsetof(scrapgpu_plan_desc, node_count) + sizeof(desc->node_count)) return invalid("plan desc is too small");
    if (desc->node_count > 0 && desc->nodes == nullptr) return invalid("plan desc has no nodes");
    std::unique_ptr<Plan> p(new Plan);
    p->hdr.backend = &kVtable;
    p->dev = d;
    for (size_t i = 0; i < desc->node_count; ++i) {
        const scrapgpu_op_desc & op = desc->nodes[i].op;
        const char * reason = nullptr;
        const scrapgpu_status st = api_supports(d, &op, &reason);
        if (st != SCRAPGPU_STATUS_OK) {
            plan_release(p.get());
            return st;
        }
        PlanNode node;
        node.op = op;
        node.in.assign(op.inputs, op.inputs + op.input_count);
        node.out.assign(op.outputs, op.outputs + op.output_count);
        if (op.params && op.params_size) {
            const uint8_t * pp = static_cast<const uint8_t *>(op.params);
            node.params.assign(pp, pp + op.params_size);
        }
        for (const auto * list : {&node.in, &node.out}) {
            for (const scrapgpu_tensor_desc & t : *list) {
                Buffer * b = buf_of(t.buffer);
                if (b == nullptr || b->dev != d) {
                    plan_release(p.get());
                    return invalid("a plan tensor is not in a buffer of the plan's device");
                }
                b->plan_refs.fetch_add(1);
                p->buffers.push_back(b);
            }
        }
        p->nodes.push_back(std::move(node));
    }
    for (PlanNode & n : p->nodes) {
        n.op.inputs = n.in.data();
        n.op.outputs = n.out.data();
        n.op.params = n.params.empty() ? nullptr : n.params.data();
    }
    // runs of MUL_MAT_IDs sharing x and ids (a MoE layer's gate and up) become one launch, runs of
    // MUL_MATs sharing x (q/k/v, gate/up issued one by one) one MUL_MAT_MULTI
    for (size_t i = 0; i < p->nodes.size();) {
        int f = 0;
        while (f < 2 && i + f + 1 < p->nodes.size() &&
               (id_fusable(&p->nodes[i], f + 1, p->nodes[i + f + 1], (int) d->cus) || mm_fusable(&p->nodes[i], f + 1, p->nodes[i + f + 1]))) {
            ++f;
        }
        p->nodes[i].fuse = f;
        i += (size_t) f + 1;
    }
    *out = reinterpret_cast<scrapgpu_plan_t *>(p.release());
    return SCRAPGPU_STATUS_OK;
}

void plan_drop_graph(Plan * p) {
    if (p->exec) hipGraphExecDestroy(p->exec);
    if (p->graph) hipGraphDestroy(p->graph);
    p->exec = nullptr;
    p->graph = nullptr;
    p->exec_stream = nullptr;
}

bool graphs_enabled() {
    static const bool on = [] {
        const char * v = std::getenv("SCRAPGPU_HIP_GRAPH");
        return v == nullptr || v[0] != '0';
    }();
    return on;
}

// scratch every node of the plan needs on this stream (allocated before a recording: no
// allocation or synchronization may happen while the stream records)
scrapgpu_status plan_prepare(Stream * s, Plan * p) {
    size_t need = 0;
    for (PlanNode & n : p->nodes) {
        if (n.op.op == SCRAPGPU_OP_MUL_MAT_ID) {
            sgk::MatArgs a;
            sgk::IdArgs id;
            if (mul_mat_id_rule(n.op.inputs[0], n.op.inputs[1], n.op.inputs[2], n.op.outputs[0], &a, &id, nullptr) == SCRAPGPU_STATUS_OK &&
                mul_mat_id_grouped(a, id)) {
                need = std::max(need, sgk::mul_mat_id_scratch_bytes(a, id));
            }
            continue;
        }
        if (n.op.op != SCRAPGPU_OP_MUL_MAT && n.op.op != SCRAPGPU_OP_MUL_MAT_MULTI) continue;
        {
            // decode with several columns: the x planes (and K-chunk partial sums) of the launch
            // over the node's weights, and of each weight alone
            sgk::MatArgs mats[3];
            int cnt = 0;
            const int total = n.op.op == SCRAPGPU_OP_MUL_MAT ? n.fuse + 1 : (int) n.op.output_count;
            for (int k = 0; k < total && k < 3; ++k) {
                const scrapgpu_op_desc & op = n.op.op == SCRAPGPU_OP_MUL_MAT ? (&n)[k].op : n.op;
                const int wi = n.op.op == SCRAPGPU_OP_MUL_MAT ? 0 : k;
                const scrapgpu_tensor_desc & x = n.op.op == SCRAPGPU_OP_MUL_MAT ? op.inputs[1] : op.inputs[op.output_count];
                sgk::MatArgs a;
                std::memset(&a, 0, sizeof(a));
                if (mul_mat_rule(op.inputs[wi], x, op.outputs[n.op.op == SCRAPGPU_OP_MUL_MAT ? 0 : k], 1, &a, nullptr) != SCRAPGPU_STATUS_OK) continue;
                if (a.N > matvec_max_n(a)) continue;
                mats[cnt++] = a;
                need = std::max(need, sgk::matvec_scratch_bytes(&a, 1));
            }
            if (cnt > 1) need = std::max(need, sgk::matvec_scratch_bytes(mats, cnt));
        }
        if (n.op.op == SCRAPGPU_OP_MUL_MAT && n.fuse > 0) {
            // MUL_MATs fused into one MULTI: the prefill launch over all their rows
            sgk::MatArgs all;
            std::memset(&all, 0, sizeof(all));
            for (int k = 0; k <= n.fuse; ++k) {
                const PlanNode & m = (&n)[k];
                sgk::MatArgs a;
                std::memset(&a, 0, sizeof(a));
                if (mul_mat_rule(m.op.inputs[0], m.op.inputs[1], m.op.outputs[0], 0, &a, nullptr) != SCRAPGPU_STATUS_OK) break;
                if (k == 0) all = a;
                else all.M += a.M;
            }
            if (all.N > matvec_max_n(all)) need = std::max(need, sgk::matmul_scratch_bytes(all, (int) s->dev->cus));
        }
        const size_t cnt = n.op.op == SCRAPGPU_OP_MUL_MAT ? 1 : n.op.output_count;
        sgk::MatArgs all;
        std::memset(&all, 0, sizeof(all));
        for (size_t i = 0; i < cnt; ++i) {
            sgk::MatArgs a;
            std::memset(&a, 0, sizeof(a));
            const scrapgpu_tensor_desc & x = n.op.op == SCRAPGPU_OP_MUL_MAT ? n.op.inputs[1] : n.op.inputs[cnt];
            if (mul_mat_rule(n.op.inputs[i], x, n.op.outputs[i], 1, &a, nullptr) == SCRAPGPU_STATUS_OK && a.N > matvec_max_n(a)) {
                need = std::max(need, sgk::matmul_scratch_bytes(a, (int) s->dev->cus));
                // a prefill MULTI may run as one launch over all its rows (run_products)
                if (all.M == 0) all = a;
                else all.M += a.M;
                if (i + 1 == cnt && cnt > 1) need = std::max(need, sgk::matmul_scratch_bytes(all, (int) s->dev->cus));
            }
        }
    }
    return need ? ensure_scratch(s, need) : SCRAPGPU_STATUS_OK;
}

scrapgpu_status api_plan_execute(scrapgpu_stream_t * stream, scrapgpu_plan_t * plan) {
    Stream * s = stream_of(stream);
    Plan * p = as<Plan>(plan);
    if (s == nullptr || p == nullptr) return invalid("not a hip stream or plan");
    if (p->dev != s->dev) return invalid("the plan was built for another device than the stream's");
    SG_HIP(use(s->dev), "hipSetDevice");
    // eager while the per-kernel profiler is on (its events are host-side records) or graphs are off
    if (!graphs_enabled() || g_prof.load(std::memory_order_relaxed) || p->nodes.empty()) {
        for (size_t i = 0; i < p->nodes.size(); i += (size_t) p->nodes[i].fuse + 1) {
            const scrapgpu_status st = exec_node(s, &p->nodes[i]);
            if (st != SCRAPGPU_STATUS_OK) return st;
        }
        return SCRAPGPU_STATUS_OK;
    }
    scrapgpu_status st = plan_prepare(s, p);
    if (st != SCRAPGPU_STATUS_OK) return st;
    if (p->exec == nullptr || p->exec_stream != s || p->exec_gen != s->scratch_gen) {
        // a graph recorded for another stream may still run there: wait for the device before
        // destroying it (the same stream with new scratch was synchronized when it grew)
        if (p->exec != nullptr && p->exec_stream != s) SG_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
        plan_drop_graph(p);
        SG_HIP(hipStreamBeginCapture(s->s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        for (size_t i = 0; i < p->nodes.size(); i += (size_t) p->nodes[i].fuse + 1) {
            st = exec_node(s, &p->nodes[i]);
            if (st != SCRAPGPU_STATUS_OK) break;
        }
        hipGraph_t g = nullptr;
        const hipError_t ec = hipStreamEndCapture(s->s, &g);
        if (st != SCRAPGPU_STATUS_OK) {
            if (g) hipGraphDestroy(g);
            return st;
        }
        if (ec != hipSuccess) return hip_fail(ec, "hipStreamEndCapture");
        const hipError_t ei = hipGraphInstantiate(&p->exec, g, nullptr, nullptr, 0);
        if (ei != hipSuccess) {
            hipGraphDestroy(g);
            p->exec = nullptr;
            return hip_fail(ei, "hipGraphInstantiate");
        }
        p->graph = g;
        p->exec_stream = s;
        p->exec_gen = s->scratch_gen;
    }
    SG_HIP(hipGraphLaunch(p->exec, s->s), "hipGraphLaunch");
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status api_plan_free(scrapgpu_plan_t * plan) {
    Plan * p = as<Plan>(plan);
    if (p == nullptr) return invalid("not a hip plan");
    if (p->exec) {
        // the recording stream may be gone already: wait for the device before dropping the graph
        if (use(p->dev) == hipSuccess) hipDeviceSynchronize();
        plan_drop_graph(p);
    }
    plan_release(p);
    delete p;
    return SCRAPGPU_STATUS_OK;
}

const scrapgpu_backend_vtable kVtable = {
    sizeof(scrapgpu_backend_vtable),
    "hip",
    nullptr,
    api_device_count,
    api_get_device,
    api_device_info,
    api_buffer_alloc,
    api_buffer_free,
    api_buffer_write,
    api_buffer_read,
    api_buffer_copy,
    api_buffer_fill,
    api_stream_sync,
    api_op_supported,
    api_plan_build,
    api_plan_execute,
    api_plan_free,
    api_stream_create,
    api_stream_free,
    api_tensor_upload,
    api_tensor_download,
    api_op_execute,
    api_stream_device,
};

// ---- device-side weight conversion (extensions) ----------------------------------------------------

scrapgpu_status convert_check(Stream * s, const scrapgpu_tensor_desc & q, const scrapgpu_tensor_desc & f) {
    if (s == nullptr) return invalid("not a hip stream");
    if (!sg::is_quant(q.dtype)) return unsupported("the quantized tensor must be Q4_0 / Q8_0 / Q4_K / Q6_K");
    if (f.dtype != SCRAPGPU_DTYPE_F32 || f.layout != SCRAPGPU_LAYOUT_NATURAL) return unsupported("the float tensor must be F32 in the natural layout");
    for (int i = 0; i < 4; ++i)
        if (sg::dim1(q.ne[i]) != sg::dim1(f.ne[i])) return invalid("the two tensors must have the same shape");
    if (sg::dim1(q.ne[0]) % (int64_t) sg::block_size(q.dtype) != 0) return invalid("rows must hold whole blocks");
    if (q.layout == SCRAPGPU_LAYOUT_R32 ? !sg::r32_eligible(q) : !sg::contiguous_ggml(q)) return unsupported("the quantized tensor must be contiguous");
    if (!sg::contiguous_ggml(f)) return unsupported("the float tensor must be contiguous");
    return SCRAPGPU_STATUS_OK;
}

// runs `body(nat_chunk_ptr, rows)` over chunks of whole row groups of every slice, packing or
// unpacking R32 around it
template <typename F>
scrapgpu_status over_chunks(Stream * s, const scrapgpu_tensor_desc & q, uint8_t * qdev, bool pack_after, F body) {
    const int64_t K = sg::dim1(q.ne[0]), M = sg::dim1(q.ne[1]);
    const int64_t slices = sg::dim1(q.ne[2]) * sg::dim1(q.ne[3]);
    const sg::R32Geom g = sg::r32_geometry(q.dtype, K, M);
    const bool r32 = q.layout == SCRAPGPU_LAYOUT_R32;
    std::lock_guard<std::mutex> lock(s->dev->mu);
    if (r32) {
        const scrapgpu_status st = ensure_staging(s->dev);
        if (st != SCRAPGPU_STATUS_OK) return st;
    }
    const int64_t chunk = r32 ? std::max<int64_t>(32, std::min<int64_t>((int64_t) (s->dev->staging_size / g.rowb) / 32 * 32, 32 * 65535)) : M;
    for (int64_t sl = 0; sl < slices; ++sl) {
        uint8_t * slice = qdev + (uint64_t) sl * M * g.rowb;
        for (int64_t rA = 0; rA < M; rA += chunk) {
            const int64_t rows = std::min(chunk, M - rA);
            uint8_t * nat = r32 ? s->dev->staging : slice + (uint64_t) rA * g.rowb;
            if (r32 && !pack_after) SG_HIP(sgk::launch_r32_move(q.dtype, K, M, rA, rows, nat, slice, false, s->s), "R32 unpack");
            const scrapgpu_status st = body(nat, sl * M + rA, rows);
            if (st != SCRAPGPU_STATUS_OK) return st;
            if (r32 && pack_after) SG_HIP(sgk::launch_r32_move(q.dtype, K, M, rA, rows, nat, slice, true, s->s), "R32 pack");
        }
    }
    // the staging buffer is free for the next caller once the stream has drained
    SG_HIP(hipStreamSynchronize(s->s), "conversion");
    return SCRAPGPU_STATUS_OK;
}

} // namespace

namespace {

// true when the core currently lists this backend's devices (public API only, so the backend also
// registers into a core it was not built with)
bool core_lists_our_devices() {
    const size_t n = scrapgpu_get_device_count();
    for (size_t i = 0; i < n; ++i) {
        scrapgpu_device_t * d = nullptr;
        if (scrapgpu_get_device(i, &d) == SCRAPGPU_STATUS_OK && dev_of(d) != nullptr) return true;
    }
    return false;
}

} // namespace

extern "C" {

scrapgpu_status scrapgpu_hip_register(void) {
    Registry & r = registry();
    std::lock_guard<std::mutex> lock(r.mu);
    if (r.registered) {
        // the devices are probed once; the vtable is registered again after
        // scrapgpu_unregister_all_backends()
        if (r.devices.empty() || core_lists_our_devices()) return SCRAPGPU_STATUS_OK;
        return scrapgpu_register_backend(&kVtable);
    }
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess && e != hipErrorNoDevice) return hip_fail(e, "hipGetDeviceCount");
    if (e == hipErrorNoDevice) n = 0;
    std::vector<int> allow;
    if (const char * env = std::getenv("SCRAPGPU_HIP_DEVICES")) {
        for (const char * p = env; *p;) {
            char * end = nullptr;
            const long v = std::strtol(p, &end, 10);
            if (end == p) break;
            allow.push_back((int) v);
            p = *end == ',' ? end + 1 : end;
        }
    }
    int rt = 0, cur = 0;
    hipRuntimeGetVersion(&rt);
    const bool had_cur = hipGetDevice(&cur) == hipSuccess;
    for (int i = 0; i < n; ++i) {
        if (!allow.empty() && std::find(allow.begin(), allow.end(), i) == allow.end()) continue;
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, i) != hipSuccess) continue;
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) continue; // kernels are built for gfx950 only
        std::unique_ptr<Device> d(new Device);
        d->hdr.backend = &kVtable;
        d->ordinal = i;
        d->name = prop.name;
        d->arch = std::string("gcnArchName ") + prop.gcnArchName;
        d->driver = "HIP runtime " + std::to_string(rt);
        d->tuning = "gfx950";
        d->total_mem = prop.totalGlobalMem;
        d->lds = prop.sharedMemPerBlock;
        d->cus = (uint32_t) prop.multiProcessorCount;
        // this device's copy of the static scratch (scrapgpu_hip_op_execute_static refuses to run
        // where the lookup failed)
        void * sp = nullptr;
        if (hipSetDevice(i) == hipSuccess && hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)) == hipSuccess) d->static_scratch = static_cast<uint8_t *>(sp);
        void * ap = nullptr;
        if (d->static_scratch != nullptr && hipGetSymbolAddress(&ap, HIP_SYMBOL(arrive_counts)) == hipSuccess) d->static_arrive = static_cast<uint32_t *>(ap);
        r.devices.push_back(std::move(d));
    }
    if (had_cur) hipSetDevice(cur); // (the static scratch lookups made each device current in turn)
    if (const char * env = std::getenv("SCRAPGPU_HIP_PROFILE")) g_prof.store(env[0] == '1');
    r.registered = true;
    const scrapgpu_status st = scrapgpu_register_backend(&kVtable);
    if (st != SCRAPGPU_STATUS_OK) r.registered = false;
    return st;
}

scrapgpu_status scrapgpu_hip_quantize(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * src, const scrapgpu_tensor_desc * dst) {
    Stream * s = stream_of(stream);
    if (s == nullptr || src == nullptr || dst == nullptr) return invalid("a null stream, src or dst");
    const scrapgpu_tensor_desc f = load_desc(*src), q = load_desc(*dst);
    scrapgpu_status st = convert_check(s, q, f);
    if (st != SCRAPGPU_STATUS_OK) return st;
    uint8_t *pf, *pq;
    if ((st = resolve(s->dev, f, &pf, "src")) != SCRAPGPU_STATUS_OK) return st;
    if ((st = resolve(s->dev, q, &pq, "dst")) != SCRAPGPU_STATUS_OK) return st;
    SG_HIP(use(s->dev), "hipSetDevice");
    const int64_t K = sg::dim1(q.ne[0]);
    const int64_t bpr = K / (int64_t) sg::block_size(q.dtype);
    const float * fp = reinterpret_cast<const float *>(pf);
    return over_chunks(s, q, pq, true, [&](uint8_t * nat, int64_t row, int64_t rows) -> scrapgpu_status {
        SG_HIP(sgk::launch_quantize(q.dtype, fp + row * K, nat, rows * bpr, s->s), "quantize");
        return SCRAPGPU_STATUS_OK;
    });
}

scrapgpu_status scrapgpu_hip_dequantize(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * src, const scrapgpu_tensor_desc * dst) {
    Stream * s = stream_of(stream);
    if (s == nullptr || src == nullptr || dst == nullptr) return invalid("a null stream, src or dst");
    const scrapgpu_tensor_desc q = load_desc(*src), f = load_desc(*dst);
    scrapgpu_status st = convert_check(s, q, f);
    if (st != SCRAPGPU_STATUS_OK) return st;
    uint8_t *pf, *pq;
    if ((st = resolve(s->dev, f, &pf, "dst")) != SCRAPGPU_STATUS_OK) return st;
    if ((st = resolve(s->dev, q, &pq, "src")) != SCRAPGPU_STATUS_OK) return st;
    SG_HIP(use(s->dev), "hipSetDevice");
    const int64_t K = sg::dim1(q.ne[0]);
    const int64_t bpr = K / (int64_t) sg::block_size(q.dtype);
    float * fp = reinterpret_cast<float *>(pf);
    return over_chunks(s, q, pq, false, [&](uint8_t * nat, int64_t row, int64_t rows) -> scrapgpu_status {
        SG_HIP(sgk::launch_dequantize(q.dtype, nat, fp + row * K, rows * bpr, s->s), "dequantize");
        return SCRAPGPU_STATUS_OK;
    });
}

scrapgpu_status scrapgpu_hip_fill_normal(scrapgpu_stream_t * stream, const scrapgpu_tensor_desc * desc, uint64_t seed, float mean, float stddev) {
    Stream * s = stream_of(stream);
    if (s == nullptr || desc == nullptr) return invalid("stream or desc is null");
    const scrapgpu_tensor_desc t = load_desc(*desc);
    if (t.dtype != SCRAPGPU_DTYPE_F32 || !sg::contiguous_ggml(t)) return unsupported("fill_normal needs a contiguous F32 tensor");
    uint8_t * p;
    scrapgpu_status st = resolve(s->dev, t, &p, "tensor");
    if (st != SCRAPGPU_STATUS_OK) return st;
    SG_HIP(use(s->dev), "hipSetDevice");
    const int64_t n = (int64_t) (sg::nbytes(t) / 4);
    SG_HIP(sgk::launch_fill_normal(reinterpret_cast<float *>(p), n, seed, mean, stddev, s->s), "fill_normal");
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status scrapgpu_hip_profile_enable(int enable) {
    g_prof.store(enable != 0);
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status scrapgpu_hip_profile_reset(void) {
    prof_collect();
    std::lock_guard<std::mutex> lock(g_prof_mu);
    g_prof_table.clear();
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status scrapgpu_hip_profile_read(size_t index, const char ** name, uint64_t * launches, double * total_ms, double * bytes, double * flops) {
    prof_collect();
    std::lock_guard<std::mutex> lock(g_prof_mu);
    if (index >= g_prof_table.size()) return invalid("no profile entry at this index");
    const ProfEntry & e = g_prof_table[index];
    if (name) *name = e.name.c_str();
    if (launches) *launches = e.launches;
    if (total_ms) *total_ms = e.ms;
    if (bytes) *bytes = e.bytes;
    if (flops) *flops = e.flops;
    return SCRAPGPU_STATUS_OK;
}

scrapgpu_status scrapgpu_hip_op_execute_static(scrapgpu_stream_t * stream, const scrapgpu_op_desc * desc) {
    Stream * s = stream_of(stream);
    if (s == nullptr) return invalid("not a hip stream");
    if (desc == nullptr) return invalid("op desc is null");
    if (s->dev->static_scratch == nullptr || s->dev->static_arrive == nullptr) {
        return set_err(SCRAPGPU_STATUS_BACKEND_ERROR, "the static scratch of this device could not be located (hipGetSymbolAddress failed at registration)");
    }
    t_static_scratch = s->dev->static_scratch;
    t_static_arrive = s->dev->static_arrive;
    const scrapgpu_status st = exec_desc(s, desc);
    t_static_scratch = nullptr;
    t_static_arrive = nullptr;
    return st;
}

scrapgpu_status scrapgpu_hip_last_launch(char * form, size_t capacity, uint64_t * grid) {
    const sgk::LaunchForm & f = sgk::last_form();
    if (form != nullptr && capacity > 0) {
        std::strncpy(form, f.form, capacity - 1);
        form[capacity - 1] = '\0';
    }
    if (grid != nullptr) *grid = f.grid;
    return SCRAPGPU_STATUS_OK;
}

void * scrapgpu_hip_stream_native(scrapgpu_stream_t * stream) {
    Stream * s = stream_of(stream);
    return s ? static_cast<void *>(s->s) : nullptr;
}

}
