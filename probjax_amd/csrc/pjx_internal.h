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

// Fills n 32-bit words at p with `value` on `stream` (a kernel, so that a
// caller may capture it in a graph); for the results of zero-length inputs
// (output 0, LSE +inf).  p may be null when n == 0.  Returns a PJX_* status.
int fill_u32(void* p, uint32_t value, size_t n, hipStream_t stream, const char* who);
// Fills n 16-bit elements with zero (n may be odd).
int zero_u16(void* p, size_t n, hipStream_t stream, const char* who);

constexpr uint32_t kPosInfBits = 0x7f800000u;  // float +inf

// Attention with no keys: every one of the o_elems output elements (fp32 if
// f32, else 16-bit) is 0 and each of the `rows` LSE entries +inf (lse may be
// null), the reference's l == 0 rule (attention_xla.py, output 0 and LSE
// +inf for rows without a valid key).
int write_keyless(void* o, float* lse, size_t o_elems, bool f32, size_t rows, hipStream_t stream,
                  const char* who);

}  // namespace pjx
