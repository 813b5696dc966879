// Core-internal routing of public calls to the backend that owns an object.
//
// Contract (reference include/scrapgpu/backend.h:21-59): every object a backend hands out begins
// with a scrapgpu_object_header whose `backend` points at the table the backend registered. The
// core keeps its own copy of each registered table, padded to the current ABI (entries past the
// caller's struct_size are null), and always calls through that copy, so a backend built against
// an older, shorter table is never read past its end.
#pragma once

#include "scrapgpu/backend.h"

namespace sgcore {

// The table that owns `obj`: the registered copy of its header's table, or (a table no longer or
// never registered) a padded copy of the header's own table. Null `obj`, a null table or one
// below the ABI 0.2 size: nullptr, with the last error set. The returned table stays valid until
// the process ends.
const scrapgpu_backend_vtable * owner_table(const void * obj, const char * call, const char * what);

// Sets the last error and returns INVALID_ARGUMENT: "<call>: <what> is null".
scrapgpu_status null_argument(const char * call, const char * what);

// Sets the last error and returns UNSUPPORTED: "<call>: backend '<name>' does not implement <entry>".
scrapgpu_status not_implemented(const char * call, const scrapgpu_backend_vtable * table, const char * entry);

} // namespace sgcore
