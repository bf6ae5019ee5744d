// fp32 flash attention at head dim 256: forward, dQ and dK/dV on
// v_mfma_f32_16x16x4f32 (full fp32 products, the 1e-5 bar).
//
// The reference's fused route takes float32 with head dims up to 256
// (probjax/nn/layers/attention.py:1187, 1193-1195).  The fp32 kernels of
// flash_fwd.hip / flash_bwd_kernels.h hold half rows of 32 queries (or keys)
// per lane on v_mfma_f32_32x32x2f32, which at D = 256 needs more than a wave's
// 512 registers; these hold 16 rows per wave instead:
//   * 16x16x4 MFMA layouts (lane l = 16*q4 + c16): A lane l holds
//     A[c16][q4], B lane l holds B[q4][c16], C lane l holds C[4*q4 + i][c16]
//     in register i.  Products contracting the head dim take dims
//     16m + 4*q4 + e in step (m, e), so each lane's operands are float4 loads
//     of 4 consecutive dims of one row; products contracting keys (queries)
//     pair the k index q4 with the key (query) 4*q4 + i of register i, so
//     their B operand is a score register as it stands and their A operand
//     one float per lane (16 lanes read 16 consecutive dims of one row).
//   * Operands come straight from global memory (L2), with no LDS staging and
//     no barriers: every wave runs independently over its own rows' keys.
//   * Masks are evaluated per score from the row's (or key's) interval
//     (row_bounds / key_bounds: causal, windows, prefix, sequence and KV
//     lengths, QKVLengthMask), plus segment ids / per-row key counts and the
//     score modifiers when MODS; the dense bias is added per score.
// Math as the other flash kernels: s = sm_scale * q.k [modified] [+ bias],
// online softmax in exp2 units (forward); p = exp2(s log2e - lse log2e),
// ds = p (dp - delta) sm_scale [* f'(s)] (backward), no roundings.
#include "flash_bwd_kernels.h"

namespace pjx {

constexpr int kWideRows = 16;      // query rows (keys) per wave
constexpr int kWideBlock = 64;     // per workgroup (4 waves)

__device__ __forceinline__ f32x4 mfma16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Score of query q, key k from the raw product x = q.k: sm_scale * x with the
// score modifiers and the dense bias `add`; g receives f'(s).  Returns the
// score in natural units.
template <bool MODS>
__device__ __forceinline__ float f32w_score(const FlashArgs& a, const HeadMods& hm, float x, float add, int q,
                                            int k, float& g) {
  const float s = x * a.scale;
  if constexpr (MODS) {
    return a.m.softcap > 0.f ? modify_score<true>(a.m, hm, s, add, q, k, g)
                             : modify_score<false>(a.m, hm, s, add, q, k, g);
  }
  g = 1.f;
  return s + add;
}

// Segment ids / per-row key counts (MODS): whether query q (id or count
// segq) keeps key k.
__device__ __forceinline__ bool f32w_seg_keep(const FlashArgs& a, int b, int segq, int k) {
  if (!a.m.seg_q) return true;
  if (a.m.seg_lt) return k < segq;
  return segq == a.m.seg_k[(size_t)b * a.Lk + k];
}

// ---------------------------------------------------------------------------
// Forward: one workgroup per (64-row query block, batch, head), heaviest
// causal block first; wave w owns rows 16w .. 16w+15 of it and walks 16-key
// blocks over its rows' key range.  S^T = K Q^T (keys as MFMA rows: lane
// holds 4 keys of one query), online softmax per query, O^T += V^T P^T.
// ---------------------------------------------------------------------------
template <int D, bool HB, bool MODS>
__global__ __launch_bounds__(256, 1) void flash_fwd_f32_wide_kernel(FlashArgs a) {
  constexpr int NM = D / 16;  // float4 groups of a row per lane; also 16-dim output blocks
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c16 = lane & 15, q4 = lane >> 4;
  const int BH = a.B * a.Hq;
  const int bh = blockIdx.x % BH;
  const int nqt = (a.Lq + kWideBlock - 1) / kWideBlock;
  const int qt = nqt - 1 - (int)(blockIdx.x / BH);
  const int b = bh / a.Hq, h = bh % a.Hq, hkv = h / (a.Hq / a.Hkv);
  const int qw = qt * kWideBlock + kWideRows * w;
  const int q = qw + c16;
  const bool row_in = q < a.Lq;
  const int q_hi = min(a.Lq, a.q_valid);
  int kv_end = min(a.Lk, a.kv_valid);
  if (a.kv_lengths) kv_end = min(kv_end, max(a.kv_lengths[b], 0));
  int lo, hi, lo0, hi0, lo1, hi1;
  row_bounds(a.m, a.causal, b, kv_end, q_hi, q, lo, hi);
  row_bounds(a.m, a.causal, b, kv_end, q_hi, qw, lo0, hi0);
  row_bounds(a.m, a.causal, b, kv_end, q_hi, min(qw + kWideRows - 1, q_hi - 1), lo1, hi1);
  const int k_begin = qw < q_hi ? (max(lo0, 0) & ~(kWideRows - 1)) : 0;
  const int k_end = qw < q_hi ? max(min(hi1 + 1, kv_end), 0) : 0;

  f32x4 qf[NM];
  {
    const float* qrow = (const float*)a.q + ((size_t)(b * a.Lq + (row_in ? q : 0)) * a.Hq + h) * D + 4 * q4;
#pragma unroll
    for (int m = 0; m < NM; ++m) qf[m] = row_in ? *(const f32x4*)(qrow + 16 * m) : f32x4{};
  }
  const size_t kv_tok = (size_t)a.Hkv * D;
  const float* Kb = (const float*)a.k + ((size_t)b * a.Lk * a.Hkv + hkv) * D;
  const float* Vb = (const float*)a.v + ((size_t)b * a.Lk * a.Hkv + hkv) * D;
  const float* brow = nullptr;
  if constexpr (HB)
    brow = a.bias + (size_t)b * a.bias_bstride + (size_t)h * a.bias_hstride + (size_t)(row_in ? q : 0) * a.Lk;
  const bool bias_vec = (a.Lk & 3) == 0;
  HeadMods hm = {0.f, 1.f};
  int segq = 0;
  if constexpr (MODS) {
    hm = head_mods(a.m, h);
    if (a.m.seg_q && row_in) segq = a.m.seg_q[(size_t)b * a.Lq + q];
  }

  f32x4 acc[NM];
#pragma unroll
  for (int i = 0; i < NM; ++i) acc[i] = f32x4{};
  float m_run = kMaxInit, l_run = 0.f;
  for (int k0 = k_begin; k0 < k_end; k0 += kWideRows) {
    // s[i] = q.k for key k0 + 4*q4 + i, query q
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    {
      const int kr = k0 + c16;
      const bool kok = kr < k_end;
      const float* kp = Kb + (size_t)(kok ? kr : 0) * kv_tok + 4 * q4;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        const f32x4 kf = kok ? *(const f32x4*)(kp + 16 * m) : f32x4{};
#pragma unroll
        for (int e = 0; e < 4; ++e) s = mfma16x16x4(kf[e], qf[m][e], s);
      }
    }
    const int kk = k0 + 4 * q4;
    f32x4 add = {0.f, 0.f, 0.f, 0.f};
    if constexpr (HB) {
      if (row_in) add = bias_vec ? load_bias4<true>(brow, kk, a.Lk) : load_bias4<false>(brow, kk, a.Lk);
    }
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = kk + i;
      float g;
      const float x = f32w_score<MODS>(a, hm, s[i], add[i], q, k, g);
      bool keep = k >= lo && k <= hi;
      if constexpr (MODS) keep = keep && f32w_seg_keep(a, b, segq, k);
      sc[i] = keep ? x * kLog2e : -INFINITY;
    }
    float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    mx = xor32_max(xor16_max(mx));
    const float m_new = fmaxf(m_run, mx);
    const float corr = fast_exp2(m_run - m_new);
    m_run = m_new;
    float p[4], rs = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = fast_exp2(sc[i] - m_new);
      rs += p[i];
    }
    l_run = fmaf(l_run, corr, rs);
#pragma unroll
    for (int db = 0; db < NM; ++db) acc[db] *= corr;
    // O^T[dim 16db + 4*q4 + r][q] += V[key kk + i][dim 16db + c16] * p[i]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = kk + i;
      const float* vp = Vb + (size_t)(k < k_end ? k : 0) * kv_tok + c16;
#pragma unroll
      for (int db = 0; db < NM; ++db) acc[db] = mfma16x16x4(k < k_end ? vp[16 * db] : 0.f, p[i], acc[db]);
    }
  }

  const float l_tot = xor32_sum(xor16_sum(l_run));
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  // acc[db][r] = O^T[dim 16db + 4*q4 + r][query q]: this lane writes dims
  // 16db + 4*q4 .. +3 of its own row.
  if (row_in) {
    float* orow = (float*)a.o + ((size_t)(b * a.Lq + q) * a.Hq + h) * D + 4 * q4;
#pragma unroll
    for (int db = 0; db < NM; ++db) *(f32x4*)(orow + 16 * db) = acc[db] * inv;
    if (a.lse && q4 == 0)
      a.lse[((size_t)b * a.Hq + h) * a.Lq + q] = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : INFINITY;
  }
}

// ---------------------------------------------------------------------------
// dQ (and delta, lse*log2e for the dK/dV kernel): the forward's decomposition.
// S^T = K Q^T and dP^T = V dO^T (keys as MFMA rows), dS^T from the LSE
// residual, dQ^T += K^T dS^T.  BIAS: 0 none, 1 dense bias, 2 dense bias and
// its gradient P (dP - delta) stored per visited score.
// ---------------------------------------------------------------------------
template <int D, int BIAS, bool MODS>
__global__ __launch_bounds__(256, 1) void flash_bwd_dq_f32_wide_kernel(FlashBwdArgs ba) {
  constexpr bool HB = BIAS != 0, DB = BIAS == 2;
  constexpr int NM = D / 16;
  const FlashArgs& a = ba.f;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c16 = lane & 15, q4 = lane >> 4;
  const int BH = a.B * a.Hq;
  const int bh = blockIdx.x % BH;
  const int nqt = (a.Lq + kWideBlock - 1) / kWideBlock;
  const int qt = nqt - 1 - (int)(blockIdx.x / BH);
  const int b = bh / a.Hq, h = bh % a.Hq, hkv = h / (a.Hq / a.Hkv);
  const int qw = qt * kWideBlock + kWideRows * w;
  const int q = qw + c16;
  const bool row_in = q < a.Lq;
  const int q_hi = min(a.Lq, a.q_valid);
  int kv_end = min(a.Lk, a.kv_valid);
  if (a.kv_lengths) kv_end = min(kv_end, max(a.kv_lengths[b], 0));
  int lo, hi, lo0, hi0, lo1, hi1;
  row_bounds(a.m, a.causal, b, kv_end, q_hi, q, lo, hi);
  row_bounds(a.m, a.causal, b, kv_end, q_hi, qw, lo0, hi0);
  row_bounds(a.m, a.causal, b, kv_end, q_hi, min(qw + kWideRows - 1, q_hi - 1), lo1, hi1);
  const int k_begin = qw < q_hi ? (max(lo0, 0) & ~(kWideRows - 1)) : 0;
  const int k_end = qw < q_hi ? max(min(hi1 + 1, kv_end), 0) : 0;

  f32x4 qf[NM], dof[NM];
  float dsum = 0.f;
  {
    const size_t roff = ((size_t)(b * a.Lq + (row_in ? q : 0)) * a.Hq + h) * D + 4 * q4;
    const float* qrow = (const float*)a.q + roff;
    const float* drow = (const float*)ba.dout + roff;
    const float* orow = (const float*)a.o + roff;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      f32x4 rq = {0.f, 0.f, 0.f, 0.f}, rd = rq, ro = rq;
      if (row_in) {
        rq = *(const f32x4*)(qrow + 16 * m);
        rd = *(const f32x4*)(drow + 16 * m);
        ro = *(const f32x4*)(orow + 16 * m);
      }
      qf[m] = rq;
      dof[m] = rd;
#pragma unroll
      for (int e = 0; e < 4; ++e) dsum = fmaf(ro[e], rd[e], dsum);
    }
  }
  const float delta = xor32_sum(xor16_sum(dsum));
  const size_t lidx = ((size_t)b * a.Hq + h) * a.Lq + q;
  float lse2 = 0.f;
  if (row_in) {
    lse2 = a.lse[lidx] * kLog2e;
    if (q4 == 0) {
      ba.delta[lidx] = delta * a.scale;
      ba.lse2[lidx] = lse2;
    }
  }
  const size_t kv_tok = (size_t)a.Hkv * D;
  const float* Kb = (const float*)a.k + ((size_t)b * a.Lk * a.Hkv + hkv) * D;
  const float* Vb = (const float*)a.v + ((size_t)b * a.Lk * a.Hkv + hkv) * D;
  const float* brow = nullptr;
  if constexpr (HB)
    brow = a.bias + (size_t)b * a.bias_bstride + (size_t)h * a.bias_hstride + (size_t)(row_in ? q : 0) * a.Lk;
  const bool bias_vec = (a.Lk & 3) == 0;
  HeadMods hm = {0.f, 1.f};
  int segq = 0;
  if constexpr (MODS) {
    hm = head_mods(a.m, h);
    if (a.m.seg_q && row_in) segq = a.m.seg_q[(size_t)b * a.Lq + q];
  }

  f32x4 acc[NM];
#pragma unroll
  for (int i = 0; i < NM; ++i) acc[i] = f32x4{};
  for (int k0 = k_begin; k0 < k_end; k0 += kWideRows) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f}, dp = s;
    {
      const int kr = k0 + c16;
      const bool kok = kr < k_end;
      const float* kp = Kb + (size_t)(kok ? kr : 0) * kv_tok + 4 * q4;
      const float* vp = Vb + (size_t)(kok ? kr : 0) * kv_tok + 4 * q4;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        const f32x4 kf = kok ? *(const f32x4*)(kp + 16 * m) : f32x4{};
        const f32x4 vf = kok ? *(const f32x4*)(vp + 16 * m) : f32x4{};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s = mfma16x16x4(kf[e], qf[m][e], s);
          dp = mfma16x16x4(vf[e], dof[m][e], dp);
        }
      }
    }
    const int kk = k0 + 4 * q4;
    f32x4 add = {0.f, 0.f, 0.f, 0.f};
    if constexpr (HB) {
      if (row_in) add = bias_vec ? load_bias4<true>(brow, kk, a.Lk) : load_bias4<false>(brow, kk, a.Lk);
    }
    float ds[4];
    f32x4 dbv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = kk + i;
      float g;
      const float x = f32w_score<MODS>(a, hm, s[i], add[i], q, k, g);
      bool keep = k >= lo && k <= hi;
      if constexpr (MODS) keep = keep && f32w_seg_keep(a, b, segq, k);
      const float p = keep ? fast_exp2(fmaf(x, kLog2e, -lse2)) : 0.f;
      const float t = p * (dp[i] - delta);  // dL/d(score)
      dbv[i] = t;
      ds[i] = t * a.scale * g;
    }
    if constexpr (DB) {
      if (row_in && kk < a.Lk) {
        float* drow = ba.dbias + (((size_t)b * a.Hq + h) * a.Lq + q) * a.Lk;
        if (bias_vec && kk + 3 < a.Lk) {
          *(f32x4*)(drow + kk) = dbv;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kk + i < a.Lk) drow[kk + i] = dbv[i];
        }
      }
    }
    // dQ^T[dim 16db + 4*q4 + r][q] += K[key kk + i][dim 16db + c16] * dS[q][kk + i]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = kk + i;
      const float* kp = Kb + (size_t)(k < k_end ? k : 0) * kv_tok + c16;
#pragma unroll
      for (int db = 0; db < NM; ++db) acc[db] = mfma16x16x4(k < k_end ? kp[16 * db] : 0.f, ds[i], acc[db]);
    }
  }
  if (row_in) {
    float* drow = (float*)ba.dq + ((size_t)(b * a.Lq + q) * a.Hq + h) * D + 4 * q4;
#pragma unroll
    for (int db = 0; db < NM; ++db) *(f32x4*)(drow + 16 * db) = acc[db];
  }
}

// ---------------------------------------------------------------------------
// dK / dV: one workgroup per (64-key block, batch, KV head); wave w owns keys
// 16w .. 16w+15 of it, whose K and V rows are the B operands of S = Q K^T and
// dP = dO V^T (queries as MFMA rows: lane holds 4 queries of one key).  For
// every query head of the GQA group and every 16-query block of the keys'
// query range: dV^T += dO^T P and dK^T += Q^T dS, the group summed in fp32.
// ---------------------------------------------------------------------------
template <int D, bool HB, bool MODS>
__global__ __launch_bounds__(256, 1) void flash_bwd_dkdv_f32_wide_kernel(FlashBwdArgs ba) {
  constexpr int NM = D / 16;
  const FlashArgs& a = ba.f;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c16 = lane & 15, q4 = lane >> 4;
  const int BH = a.B * a.Hkv;
  const int bh = blockIdx.x % BH;
  const int b = bh / a.Hkv, hkv = bh % a.Hkv;
  const int G = a.Hq / a.Hkv;
  const int kw = (int)(blockIdx.x / BH) * kWideBlock + kWideRows * w;
  const int key = kw + c16;
  const bool key_in = key < a.Lk;
  const int q_hi = min(a.Lq, a.q_valid);
  int kv_end = min(a.Lk, a.kv_valid);
  if (a.kv_lengths) kv_end = min(kv_end, max(a.kv_lengths[b], 0));
  int qlo, qhi, qa0, qa1, qb0, qb1;
  key_bounds(a.m, a.causal, b, kv_end, q_hi, key, qlo, qhi);
  key_bounds(a.m, a.causal, b, kv_end, q_hi, kw, qa0, qa1);
  key_bounds(a.m, a.causal, b, kv_end, q_hi, min(kw + kWideRows - 1, kv_end - 1), qb0, qb1);
  const int q_begin = kw < kv_end ? (max(qa0, 0) & ~(kWideRows - 1)) : 0;
  const int q_end = kw < kv_end ? max(min(qb1 + 1, q_hi), 0) : 0;

  f32x4 kf[NM], vf[NM];
  {
    const size_t koff = ((size_t)(b * a.Lk + (key_in ? key : 0)) * a.Hkv + hkv) * D + 4 * q4;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      kf[m] = key_in ? *(const f32x4*)((const float*)a.k + koff + 16 * m) : f32x4{};
      vf[m] = key_in ? *(const f32x4*)((const float*)a.v + koff + 16 * m) : f32x4{};
    }
  }
  int segk = 0;
  if constexpr (MODS) {
    if (a.m.seg_k && key_in) segk = a.m.seg_k[(size_t)b * a.Lk + key];
  }
  f32x4 acck[NM], accv[NM];
#pragma unroll
  for (int i = 0; i < NM; ++i) acck[i] = accv[i] = f32x4{};

  for (int hg = 0; hg < G; ++hg) {
    const int h = hkv * G + hg;
    HeadMods hm = {0.f, 1.f};
    if constexpr (MODS) hm = head_mods(a.m, h);
    const float* Qb = (const float*)a.q + ((size_t)b * a.Lq * a.Hq + h) * D;
    const float* Ob = (const float*)ba.dout + ((size_t)b * a.Lq * a.Hq + h) * D;
    const size_t q_tok = (size_t)a.Hq * D;
    const size_t lbase = ((size_t)b * a.Hq + h) * a.Lq;
    const float* bbase = nullptr;
    if constexpr (HB) bbase = a.bias + (size_t)b * a.bias_bstride + (size_t)h * a.bias_hstride;
    for (int q0 = q_begin; q0 < q_end; q0 += kWideRows) {
      // s[i] = q.k, dp[i] = do.v for query q0 + 4*q4 + i, key `key`
      f32x4 s = {0.f, 0.f, 0.f, 0.f}, dp = s;
      {
        const int qr = q0 + c16;
        const bool qok = qr < q_end;
        const float* qp = Qb + (size_t)(qok ? qr : 0) * q_tok + 4 * q4;
        const float* op = Ob + (size_t)(qok ? qr : 0) * q_tok + 4 * q4;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          const f32x4 qv = qok ? *(const f32x4*)(qp + 16 * m) : f32x4{};
          const f32x4 ov = qok ? *(const f32x4*)(op + 16 * m) : f32x4{};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s = mfma16x16x4(qv[e], kf[m][e], s);
            dp = mfma16x16x4(ov[e], vf[m][e], dp);
          }
        }
      }
      float p[4], ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qq = q0 + 4 * q4 + i;
        const bool qok = qq < q_end;
        bool keep = qok && key_in && qq >= qlo && qq <= qhi;
        if constexpr (MODS) {
          if (keep && a.m.seg_q) {
            const int sq = a.m.seg_q[(size_t)b * a.Lq + qq];
            keep = a.m.seg_lt ? key < sq : sq == segk;
          }
        }
        float add = 0.f;
        if constexpr (HB) {
          if (keep) add = bbase[(size_t)qq * a.Lk + key];
        }
        float g;
        const float x = f32w_score<MODS>(a, hm, s[i], add, qq, key, g);
        const float l2 = qok ? ba.lse2[lbase + qq] : 0.f;
        const float dl = qok ? ba.delta[lbase + qq] : 0.f;  // delta * sm_scale
        p[i] = keep ? fast_exp2(fmaf(x, kLog2e, -l2)) : 0.f;
        ds[i] = p[i] * fmaf(dp[i], a.scale, -dl) * g;
      }
      // dV^T[dim][key] += dO[q0 + 4*q4 + i][dim] p[i];  dK^T += Q[.][dim] ds[i]
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qq = q0 + 4 * q4 + i;
        const bool qok = qq < q_end;
        const float* qp = Qb + (size_t)(qok ? qq : 0) * q_tok + c16;
        const float* op = Ob + (size_t)(qok ? qq : 0) * q_tok + c16;
#pragma unroll
        for (int db = 0; db < NM; ++db) {
          accv[db] = mfma16x16x4(qok ? op[16 * db] : 0.f, p[i], accv[db]);
          acck[db] = mfma16x16x4(qok ? qp[16 * db] : 0.f, ds[i], acck[db]);
        }
      }
    }
  }
  if (key_in) {
    const size_t koff = ((size_t)(b * a.Lk + key) * a.Hkv + hkv) * D + 4 * q4;
#pragma unroll
    for (int db = 0; db < NM; ++db) {
      *(f32x4*)((float*)ba.dk + koff + 16 * db) = acck[db];
      *(f32x4*)((float*)ba.dv + koff + 16 * db) = accv[db];
    }
  }
}

int launch_flash_f32_wide(const FlashArgs& a, hipStream_t s) {
  const long blocks = (long)((a.Lq + kWideBlock - 1) / kWideBlock) * a.B * a.Hq;
  if (blocks > 0x7fffffffL) return fail(PJX_ERR_INVALID, "pjx_flash_fwd: grid too large");
  const dim3 grid((unsigned)blocks);
  const bool hb = a.bias != nullptr, mods = a.ext != 0;
  if (mods) {
    if (hb) launch_kernel<flash_fwd_f32_wide_kernel<256, true, true>>(grid, dim3(256), 0, s, a);
    else launch_kernel<flash_fwd_f32_wide_kernel<256, false, true>>(grid, dim3(256), 0, s, a);
  } else {
    if (hb) launch_kernel<flash_fwd_f32_wide_kernel<256, true, false>>(grid, dim3(256), 0, s, a);
    else launch_kernel<flash_fwd_f32_wide_kernel<256, false, false>>(grid, dim3(256), 0, s, a);
  }
  return check_launch("pjx_flash_fwd");
}

template <bool MODS>
static void launch_dq_f32w(const FlashBwdArgs& ba, dim3 grid, hipStream_t s) {
  if (ba.dbias) launch_kernel<flash_bwd_dq_f32_wide_kernel<256, 2, MODS>>(grid, dim3(256), 0, s, ba);
  else if (ba.f.bias) launch_kernel<flash_bwd_dq_f32_wide_kernel<256, 1, MODS>>(grid, dim3(256), 0, s, ba);
  else launch_kernel<flash_bwd_dq_f32_wide_kernel<256, 0, MODS>>(grid, dim3(256), 0, s, ba);
}

template <bool MODS>
static void launch_dkdv_f32w(const FlashBwdArgs& ba, dim3 grid, hipStream_t s) {
  if (ba.f.bias) launch_kernel<flash_bwd_dkdv_f32_wide_kernel<256, true, MODS>>(grid, dim3(256), 0, s, ba);
  else launch_kernel<flash_bwd_dkdv_f32_wide_kernel<256, false, MODS>>(grid, dim3(256), 0, s, ba);
}

int run_flash_f32_wide_bwd(const FlashBwdArgs& ba, hipStream_t s) {
  const FlashArgs& a = ba.f;
  const long qb = (long)((a.Lq + kWideBlock - 1) / kWideBlock) * a.B * a.Hq;
  const long kb = (long)((a.Lk + kWideBlock - 1) / kWideBlock) * a.B * a.Hkv;
  if (qb > 0x7fffffffL || kb > 0x7fffffffL) return fail(PJX_ERR_INVALID, "pjx_flash_bwd: grid too large");
  const bool mods = a.ext != 0;
  if (a.Lq > 0) {
    if (mods) launch_dq_f32w<true>(ba, dim3((unsigned)qb), s);
    else launch_dq_f32w<false>(ba, dim3((unsigned)qb), s);
    const int rc = check_launch("pjx_flash_bwd (dq)");
    if (rc != PJX_OK) return rc;
  }
  if (a.Lk == 0) return PJX_OK;
  if (mods) launch_dkdv_f32w<true>(ba, dim3((unsigned)kb), s);
  else launch_dkdv_f32w<false>(ba, dim3((unsigned)kb), s);
  return check_launch("pjx_flash_bwd (dk, dv)");
}

}  // namespace pjx
