// Library-wide C-ABI entry points: version, error reporting.
#include <cxxabi.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>

#include "flash_common.h"

namespace pjx {

static thread_local char g_error[512];
// Kernel instances launched by the calling thread's current (or last) entry
// point call, in launch order, ';'-separated.
static thread_local char g_launches[2048];

void set_error(const char* msg) {
  strncpy(g_error, msg, sizeof(g_error) - 1);
  g_error[sizeof(g_error) - 1] = '\0';
}

void clear_error() {
  g_error[0] = '\0';
  g_launches[0] = '\0';
}

void note_launch(const char* name) {
  const size_t n = strlen(g_launches), m = strlen(name);
  if (n + m + 2 > sizeof(g_launches)) return;  // the log keeps the first launches that fit
  if (n > 0) g_launches[n] = ';';
  memcpy(g_launches + n + (n > 0), name, m + 1);
}

// typeid(KernelTag<&kern<...>>) demangles to
// "pjx::KernelTag<&(void pjx::kern<args>(params))>" for a template kernel and
// "pjx::KernelTag<&pjx::kern>" for a plain one; keeps "kern<args>" / "kern"
// without namespace qualifiers.
std::string demangled_kernel_name(const char* mangled) {
  int st = 0;
  char* d = abi::__cxa_demangle(mangled, nullptr, nullptr, &st);
  std::string full = (st == 0 && d) ? d : mangled;
  free(d);
  for (size_t p; (p = full.find("(anonymous namespace)::")) != std::string::npos;) full.erase(p, 23);
  const size_t t = full.find("KernelTag<");
  std::string name = full;
  if (t != std::string::npos) {
    const size_t e = full.rfind('>');
    name = full.substr(t + 10, e == std::string::npos || e < t + 10 ? std::string::npos : e - t - 10);
  }
  if (!name.empty() && name[0] == '&') name.erase(0, 1);
  if (!name.empty() && name[0] == '(') name.erase(0, 1);
  if (name.compare(0, 5, "void ") == 0) name.erase(0, 5);
  const size_t paren = name.find('(');
  if (paren != std::string::npos) name.erase(paren);
  for (size_t p; (p = name.find("pjx::")) != std::string::npos;) name.erase(p, 5);
  return name;
}

int check_launch(const char* where) {
  const hipError_t err = hipGetLastError();
  if (err == hipSuccess) return PJX_OK;
  char buf[512];
  snprintf(buf, sizeof(buf), "%s: kernel launch failed: %s", where, hipGetErrorString(err));
  set_error(buf);
  return PJX_ERR_LAUNCH;
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* p, uint32_t value, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = value;
}

__global__ __launch_bounds__(256) void zero_u16_kernel(uint16_t* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0;
}

int fill_u32(void* p, uint32_t value, size_t n, hipStream_t stream, const char* who) {
  if (n == 0) return PJX_OK;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 65536);
  launch_kernel<fill_u32_kernel>(dim3((unsigned)blocks), dim3(256), 0, stream, (uint32_t*)p, value, n);
  return check_launch(who);
}

int zero_u16(void* p, size_t n, hipStream_t stream, const char* who) {
  if (n == 0) return PJX_OK;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 65536);
  launch_kernel<zero_u16_kernel>(dim3((unsigned)blocks), dim3(256), 0, stream, (uint16_t*)p, n);
  return check_launch(who);
}

int write_keyless(void* o, float* lse, size_t o_elems, bool f32, size_t rows, hipStream_t stream,
                  const char* who) {
  int rc = f32 ? fill_u32(o, 0u, o_elems, stream, who) : zero_u16(o, o_elems, stream, who);
  if (rc == PJX_OK && lse) rc = fill_u32(lse, kPosInfBits, rows, stream, who);
  return rc;
}

int device_cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
    return n;
  return 256;
}

int lower_score_mods(const pjx_score_mods* mods, FlashArgs& a, const char* who) {
  ScoreMods& m = a.m;
  m.causal_shift = 0;
  m.win_left = m.win_right = kNoBound;
  m.prefix = m.seqlen = m.seg_q = m.seg_k = nullptr;
  m.seg_lt = 0;
  m.alibi = nullptr;
  m.alibi_sym = 0;
  m.softcap = 0.f;
  m.head_scale = nullptr;
  m.constant = 0.f;
  a.ext = 0;
  if (!mods) return PJX_OK;
  char buf[256];
  if (mods->softcap < 0.f || mods->softcap != mods->softcap) {
    snprintf(buf, sizeof(buf), "%s: softcap must be >= 0", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  if (mods->softcap > 0.f && mods->head_scales) {
    snprintf(buf, sizeof(buf), "%s: softcap and head_scales exclude each other", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  if ((mods->segment_q == nullptr) != (mods->segment_k == nullptr)) {
    snprintf(buf, sizeof(buf), "%s: segment_q and segment_k go together", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  if (mods->row_kv_lengths && mods->segment_q) {
    snprintf(buf, sizeof(buf), "%s: row_kv_lengths excludes segment ids (one stateful mask)", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  if (mods->window_left >= kNoBound || mods->window_right >= kNoBound ||
      mods->causal_shift >= kNoBound || mods->causal_shift <= -kNoBound) {
    snprintf(buf, sizeof(buf), "%s: window / causal_shift out of range", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  m.causal_shift = a.causal ? mods->causal_shift : 0;
  m.win_left = mods->window_left >= 0 ? mods->window_left : kNoBound;
  m.win_right = mods->window_right >= 0 ? mods->window_right : kNoBound;
  m.prefix = mods->prefix_lengths;
  m.seqlen = mods->seq_lengths;
  m.seg_q = mods->segment_q;
  m.seg_k = mods->segment_k;
  if (mods->row_kv_lengths) {
    m.seg_q = mods->row_kv_lengths;
    m.seg_k = nullptr;
    m.seg_lt = 1;
  }
  m.alibi = mods->alibi_slopes;
  m.alibi_sym = mods->alibi_symmetric ? 1 : 0;
  m.softcap = mods->softcap;
  m.head_scale = mods->head_scales;
  m.constant = mods->constant;
  const bool full = m.seg_q || m.alibi || m.softcap > 0.f || m.head_scale || m.constant != 0.f;
  const bool intervals = m.causal_shift != 0 || m.win_left != kNoBound || m.win_right != kNoBound ||
                         m.prefix || m.seqlen;
  a.ext = full ? 2 : intervals ? 1 : 0;
  return PJX_OK;
}

}  // namespace pjx

extern "C" int pjx_version(void) { return 100; }

extern "C" const char* pjx_last_error(void) { return pjx::g_error; }

extern "C" const char* pjx_last_launches(void) { return pjx::g_launches; }
