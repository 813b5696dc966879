// Core-internal queries of the backend registry (not part of the public C API).
#pragma once

#include "scrapgpu/backend.h"

// true when a backend whose device enumeration is `get_device` is currently registered
bool sg_registry_contains(size_t (*get_device_count)(void *));
