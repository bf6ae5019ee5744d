// Flash-attention backward: the launchers and the C ABI entry point
// pjx_flash_bwd.  The kernels and their description are in
// flash_bwd_kernels.h; this unit is built in the VGPR MFMA register form, the
// D = 256 dK/dV kernel in flash_bwd256.hip in the default form.
#include "flash_bwd_kernels.h"

namespace pjx {

// dQ first (it writes the delta * sm_scale and lse*log2e the dK/dV kernel reads), then
// dK/dV.  Without keys only dQ (= 0) runs; without queries only dK/dV (= 0).
template <int D, int EXT>
static int run_bwd_f32(const FlashBwdArgs& a, bool hb, hipStream_t s) {
  if (a.f.Lq > 0) {
    const bool db = a.dbias != nullptr;
    const int rc = db ? launch_dq<flash_bwd_dq_f32_kernel<D, 2, EXT>>(a, s)
                 : hb ? launch_dq<flash_bwd_dq_f32_kernel<D, 1, EXT>>(a, s)
                      : launch_dq<flash_bwd_dq_f32_kernel<D, 0, EXT>>(a, s);
    if (rc != PJX_OK) return rc;
  }
  if (a.f.Lk == 0) return PJX_OK;
  return hb ? launch_dkdv<flash_bwd_dkdv_f32_kernel<D, true, EXT>>(a, s)
            : launch_dkdv<flash_bwd_dkdv_f32_kernel<D, false, EXT>>(a, s);
}

template <typename E, int D, int EXT>
static int run_bwd_h16(const FlashBwdArgs& a, bool hb, hipStream_t s) {
  // Small grids (at most one workgroup per CU, or two with a causal mask,
  // whose tiles differ in length) run two groups of 4 waves per workgroup.
  const int cus = device_cu_count();
  auto small = [&](long blocks) { return EXT == 0 && blocks <= 2L * cus && (a.f.causal || blocks <= cus); };
  if (a.f.Lq > 0) {
    const bool db = a.dbias != nullptr;
    int rc;
    if (small((long)a.f.n_qtiles * a.f.B * a.f.Hq)) {
      constexpr int T2 = 2 * kThreads;
      rc = db ? launch_dq<flash_bwd_dq_kernel<E, D, 2, 0, 2>>(a, s, T2)
         : hb ? launch_dq<flash_bwd_dq_kernel<E, D, 1, 0, 2>>(a, s, T2)
              : launch_dq<flash_bwd_dq_kernel<E, D, 0, 0, 2>>(a, s, T2);
    } else {
      rc = db ? launch_dq<flash_bwd_dq_kernel<E, D, 2, EXT>>(a, s)
         : hb ? launch_dq<flash_bwd_dq_kernel<E, D, 1, EXT>>(a, s)
              : launch_dq<flash_bwd_dq_kernel<E, D, 0, EXT>>(a, s);
    }
    if (rc != PJX_OK) return rc;
  }
  if (a.f.Lk == 0) return PJX_OK;
  if (small((long)((a.f.Lk + kBKV - 1) / kBKV) * a.f.B * a.f.Hkv))
    return hb ? launch_dkdv<flash_bwd_dkdv_kernel<E, D, true, 0, 2>>(a, s, 2 * kThreads)
              : launch_dkdv<flash_bwd_dkdv_kernel<E, D, false, 0, 2>>(a, s, 2 * kThreads);
  return hb ? launch_dkdv<flash_bwd_dkdv_kernel<E, D, true, EXT>>(a, s)
            : launch_dkdv<flash_bwd_dkdv_kernel<E, D, false, EXT>>(a, s);
}

template <int D, int EXT>
static int run_bwd_t(const FlashBwdArgs& a, int dtype, bool hb, hipStream_t s) {
  if (dtype == PJX_DTYPE_F32) return run_bwd_f32<D, EXT>(a, hb, s);
  if (dtype == PJX_DTYPE_F16) return run_bwd_h16<F16Fmt, D, EXT>(a, hb, s);
  return run_bwd_h16<Bf16Fmt, D, EXT>(a, hb, s);
}

template <int D>
static int run_bwd(const FlashBwdArgs& a, int dtype, bool hb, hipStream_t s) {
  if (a.f.ext == 2) return run_bwd_t<D, 2>(a, dtype, hb, s);
  return a.f.ext == 1 ? run_bwd_t<D, 1>(a, dtype, hb, s) : run_bwd_t<D, 0>(a, dtype, hb, s);
}

}  // namespace pjx

using namespace pjx;

extern "C" size_t pjx_flash_bwd_workspace_size(int64_t batch, int64_t q_heads, int64_t q_len) {
  if (batch <= 0 || q_heads <= 0 || q_len <= 0) return 0;
  return (size_t)(2 * batch * q_heads * q_len) * sizeof(float);
}

extern "C" size_t pjx_flash_bwd_ds_workspace_size(int dtype, int64_t batch, int64_t q_heads, int64_t q_len,
                                                  int64_t kv_len, int64_t head_dim) {
  if (dtype != PJX_DTYPE_BF16 && dtype != PJX_DTYPE_F16) return 0;
  if (head_dim != 256) return 0;
  if (batch <= 0 || q_heads <= 0 || q_len <= 0 || kv_len <= 0) return 0;
  if (q_len > (1 << 30) || kv_len > (1 << 30)) return 0;
  return wide_bwd_ds_offset(pjx_flash_bwd_workspace_size(batch, q_heads, q_len)) +
         wide_bwd_ds_bytes(batch, q_heads, q_len, kv_len);
}

extern "C" int pjx_flash_bwd(int dtype, const void* q, const void* k, const void* v, const void* o,
                             const void* dout, const float* lse, void* dq, void* dk, void* dv,
                             float* dbias, void* workspace, size_t workspace_bytes, const int32_t* kv_lengths,
                             const float* bias, int64_t bias_batch, int64_t bias_heads,
                             int64_t batch, int64_t q_len, int64_t kv_len, int64_t q_heads,
                             int64_t kv_heads, int64_t head_dim, int64_t q_valid, int64_t kv_valid,
                             int causal, float sm_scale, const pjx_score_mods* mods, void* stream) {
  clear_error();
  if (dtype != PJX_DTYPE_BF16 && dtype != PJX_DTYPE_F16 && dtype != PJX_DTYPE_F32)
    return fail(PJX_ERR_INVALID, "pjx_flash_bwd: dtype must be PJX_DTYPE_BF16, PJX_DTYPE_F16 or PJX_DTYPE_F32");
  // zero-element tensors may come as null pointers
  const bool q_none = batch == 0 || q_len == 0, k_none = batch == 0 || kv_len == 0;
  if ((!q_none && (!q || !o || !dout || !lse || !dq)) || (!k_none && (!k || !v || !dk || !dv)))
    return fail(PJX_ERR_INVALID, "pjx_flash_bwd: q, k, v, o, dout, lse, dq, dk, dv must be non-null");
  if (batch < 0 || q_len < 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0)
    return fail(PJX_ERR_INVALID, "pjx_flash_bwd: negative or zero size");
  if (q_heads % kv_heads != 0)
    return fail(PJX_ERR_INVALID, "pjx_flash_bwd: q_heads must be a multiple of kv_heads");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(PJX_ERR_INVALID, "pjx_flash_bwd: head_dim must be 64, 128 or 256");
  if (!(sm_scale > 0.f)) return fail(PJX_ERR_INVALID, "pjx_flash_bwd: sm_scale must be > 0");
  if (bias && !((bias_batch == 1 || bias_batch == batch) && (bias_heads == 1 || bias_heads == q_heads)))
    return fail(PJX_ERR_INVALID, "pjx_flash_bwd: bias must be [1|B, 1|Hq, Lq, Lk]");
  if (dbias && !bias) return fail(PJX_ERR_INVALID, "pjx_flash_bwd: dbias needs the bias");
  const int64_t elems = std::max(batch * q_len * q_heads, batch * kv_len * kv_heads) * head_dim;
  if (elems > (int64_t)1 << 40 || q_len > (1 << 30) || kv_len > (1 << 30) ||
      (int64_t)q_heads * head_dim * 4 * 64 > 0xffffffffLL)
    return fail(PJX_ERR_INVALID, "pjx_flash_bwd: sizes out of range");
  if (batch == 0 || (q_len == 0 && kv_len == 0)) return PJX_OK;
  const bool f32 = dtype == PJX_DTYPE_F32;
  if (q_len == 0 || kv_len == 0) {
    // no query reaches a key: dK = dV = 0 (no queries) or dQ = 0 (no keys)
    hipStream_t s0 = (hipStream_t)stream;
    const char* who = "pjx_flash_bwd";
    auto zero = [&](void* p, size_t n) { return f32 ? fill_u32(p, 0u, n, s0, who) : zero_u16(p, n, s0, who); };
    if (kv_len == 0) return zero(dq, (size_t)(batch * q_len * q_heads * head_dim));
    const int rc = zero(dk, (size_t)(batch * kv_len * kv_heads * head_dim));
    return rc != PJX_OK ? rc : zero(dv, (size_t)(batch * kv_len * kv_heads * head_dim));
  }
  const size_t need = pjx_flash_bwd_workspace_size(batch, q_heads, q_len);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(PJX_ERR_WORKSPACE, "pjx_flash_bwd: workspace missing or smaller than pjx_flash_bwd_workspace_size()");

  FlashBwdArgs ba;
  FlashArgs& a = ba.f;
  a.q = q; a.k = k; a.v = v; a.o = const_cast<void*>(o); a.lse = const_cast<float*>(lse);
  a.kv_lengths = kv_lengths;
  a.bias = bias;
  a.bias_hstride = (bias && bias_heads != 1) ? q_len * kv_len : 0;
  a.bias_bstride = (bias && bias_batch != 1) ? bias_heads * q_len * kv_len : 0;
  a.B = (int)batch; a.Lq = (int)q_len; a.Lk = (int)kv_len;
  a.Hq = (int)q_heads; a.Hkv = (int)kv_heads;
  a.q_valid = (int)std::min<int64_t>(std::max<int64_t>(q_valid, 0), q_len);
  a.kv_valid = (int)std::min<int64_t>(std::max<int64_t>(kv_valid, 0), kv_len);
  a.causal = causal ? 1 : 0;
  a.f16 = dtype == PJX_DTYPE_F16;
  a.scale = sm_scale;
  a.n_qtiles = (int)((q_len + kBQ - 1) / kBQ);
  if ((long)a.n_qtiles * batch * q_heads > 0x7fffffffL ||
      (long)((kv_len + kBKV - 1) / kBKV) * batch * kv_heads > 0x7fffffffL)
    return fail(PJX_ERR_INVALID, "pjx_flash_bwd: grid too large");
  const int mrc = lower_score_mods(mods, a, "pjx_flash_bwd");
  if (mrc != PJX_OK) return mrc;
  ba.dout = dout;
  ba.delta = (float*)workspace;
  ba.lse2 = ba.delta + batch * q_heads * q_len;
  ba.dq = dq; ba.dk = dk; ba.dv = dv;
  ba.dbias = dbias;
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 256 && f32) return run_flash_f32_wide_bwd(ba, s);
  if (head_dim == 256) {
    // dQ (and delta, lse*log2e): the 16-row wide kernel.  dK/dV: with a dense
    // bias and no extended masks the 32-key kernel above at one wave per SIMD
    // (32x32x16 MFMAs; 501 registers, no spills); otherwise the wide kernels,
    // one head group per KV head (no partials): without bias or extended
    // masks the column-split one at two workgroups per CU, which is faster
    // than the 32-key kernel there.
    WideBwdArgs wa;
    wa.f = a;
    wa.f.dv = 256;
    wa.dout = dout;
    wa.delta = ba.delta;
    wa.lse2 = ba.lse2;
    wa.dq = dq; wa.dk = dk; wa.dv = dv;
    wa.dbias = dbias;
    wa.part = nullptr;
    wa.nsplit = 1;
    wa.ds = nullptr;
    wa.ds_nq32 = wa.ds_nk16 = 0;
    const size_t ds_need = pjx_flash_bwd_ds_workspace_size(dtype, batch, q_heads, q_len, kv_len, head_dim);
    if (!f32 && !bias && a.ext == 0 && ds_need > 0 && workspace_bytes >= ds_need) {
      // the dS route (flash_wide_bwd.hip): the workspace holds the dS blocks
      wa.ds = (uint16_t*)((unsigned char*)workspace + wide_bwd_ds_offset(need));
      wa.ds_nq32 = (int)wide_bwd_ds_nq32(q_len);
      wa.ds_nk16 = (int)wide_bwd_ds_nk16(kv_len);
    }
    if (a.ext != 0 || bias == nullptr) return run_wide_bwd(wa, 256, 256, false, s, "pjx_flash_bwd");
    const int rc = run_wide_bwd(wa, 256, 256, false, s, "pjx_flash_bwd", true);
    if (rc != PJX_OK) return rc;
    const bool hb256 = bias != nullptr;
    return launch_dkdv256(ba, dtype == PJX_DTYPE_F16, hb256, s);
  }
  const bool hb = bias != nullptr;
  return head_dim == 128 ? run_bwd<128>(ba, dtype, hb, s) : run_bwd<64>(ba, dtype, hb, s);
}
