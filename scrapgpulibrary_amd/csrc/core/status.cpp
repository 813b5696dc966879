// ABI version and the thread-local last error (reference src/core/status.cpp:1-39).
#include "scrapgpu/status.h"

#include <string>

namespace {
thread_local std::string t_last_error;
}

extern "C" {

uint32_t scrapgpu_get_abi_version(void) {
    return (SCRAPGPU_ABI_VERSION_MAJOR << 16) | SCRAPGPU_ABI_VERSION_MINOR;
}

const char * scrapgpu_status_string(scrapgpu_status status) {
    static const char * const names[] = {"OK", "UNSUPPORTED", "INVALID_ARGUMENT", "OUT_OF_MEMORY", "BACKEND_ERROR", "DEVICE_LOST"};
    const unsigned i = (unsigned) status;
    return i < sizeof(names) / sizeof(names[0]) ? names[i] : "UNKNOWN";
}

const char * scrapgpu_last_error(void) {
    return t_last_error.c_str();
}

void scrapgpu_clear_last_error(void) {
    t_last_error.clear();
}

void scrapgpu_set_last_error(const char * message) {
    t_last_error.assign(message == nullptr ? "" : message);
}

}
