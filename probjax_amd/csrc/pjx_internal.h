// Host-side helpers shared by the C-ABI entry points: a thread-local error
// message and launch checking.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/probjax_hip.h"

namespace pjx {

void set_error(const char* msg);
void clear_error();

inline int fail(int code, const char* msg) {
  set_error(msg);
  return code;
}

// Report a failed launch (bad configuration, out of resources) as an error
// instead of aborting.
int check_launch(const char* where);

// Compute units of the calling thread's current device, queried on every call
// (no cached state: the library holds no mutable globals besides the
// thread-local error string); 256 if the query fails.
int device_cu_count();

}  // namespace pjx
