// Host-side helpers shared by the C-ABI entry points: a thread-local error
// message and launch checking.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <typeinfo>

#include "../../include/probjax_hip.h"

namespace pjx {

void set_error(const char* msg);
void clear_error();

// The launch log behind pjx_last_launches(): clear_error() empties it, and
// every kernel launch appends the instance's name (kernel_name<K>()).
void note_launch(const char* name);
std::string demangled_kernel_name(const char* mangled);
template <auto K>
struct KernelTag {};
// "kernel<template args>" of the kernel instance K, e.g.
// "flash_fwd_bf16_pipe_kernel<Bf16Fmt, 128, 32, 3, 1>".
template <auto K>
const char* kernel_name() {
  static const std::string name = demangled_kernel_name(typeid(KernelTag<K>).name());
  return name.c_str();
}

// Notes and enqueues one launch of kernel instance K.
template <auto K, typename... Args>
inline void launch_kernel(dim3 grid, dim3 block, size_t lds, hipStream_t stream, Args... args) {
  note_launch(kernel_name<K>());
  hipLaunchKernelGGL(K, grid, block, lds, stream, args...);
}

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
