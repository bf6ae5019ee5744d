// Extended masks and score modifiers of the flash kernels (forward and
// backward), evaluated in-kernel.
//
// Positional masks.  Every positional mask of the path keeps, for query row
// q of batch b, one interval of keys [lo(q), hi(q)], and lo and hi never
// decrease as q grows; an AND of such masks is the intersection of their
// intervals (probjax/nn/pallas_kernels/attention_mask_bias.py):
//   CausalMask               hi <= q                      (:617-648)
//   CausalFromBottomRightMask hi <= q + (Lk - Lq)         (:753-782)
//   LocalWindowMask          q - left <= k <= q + right   (:651-704)
//   CausalLocalWindowMask    q - left <= k <= q           (:707-750)
//   PrefixLMMask             hi <= max(q, P[b] - 1)       (:785-868)
//   SeqLenMask               q < L[b] ? [0, L-1] : [q, q] (:1239-1398)
//   KVLenMask / QKVLengthMask / Lk                        (:1401-1532, :1079-1129)
// Monotone intervals give each tile of rows its key range from its first and
// last row, and each key its query range [qlo(k), qhi(k)] (the dK/dV kernels'
// view), so masking is two compares per score.
//
// SameSegmentMask / BlockDiagonal(Causal)Mask (:1537-1668, :871-1076) compare
// per-position segment ids on top of the interval; KeyPaddingMask
// (:1132-1236) gives each query row its own key count (k < seg_q[q], seg_lt),
// which is not monotone in q and so is checked per score like the ids.
//
// Score modifiers, applied to s = sm_scale * q.k in the order of the
// reference's SumBias composition (:553-582): one multiplicative modifier
// f(s) -- SoftCappingBias cap*tanh(s/cap) (:2564-2603) or PerHeadScaleBias
// s*scale[h] (:2606-2648) -- then the additive terms: the dense bias,
// -slope[h] * relu(q-k) or |q-k| (CausalAlibiBias :2230-2255,
// SymmetricAlibiBias :2355-2380, DistanceDecayBias :2387-2414) and a constant
// (ConstantBias :1781-1805).  The backward multiplies dS by f'(s).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pjx {

constexpr int kNoBound = 0x3fffffff;  // window side / shift absent

struct ScoreMods {
  int causal_shift;      // with causal: k <= q + causal_shift
  int win_left;          // kNoBound: none
  int win_right;         // kNoBound: none
  const int32_t* prefix; // [B] PrefixLM lengths or null
  const int32_t* seqlen; // [B] SeqLenMask lengths or null
  const int32_t* seg_q;  // [B, Lq] segment ids (or row key lengths) or null
  const int32_t* seg_k;  // [B, Lk]; null with seg_lt
  int seg_lt;            // 0: keep seg_q[q] == seg_k[k]; 1: keep k < seg_q[q]
  const float* alibi;    // [Hq] slopes or null
  int alibi_sym;         // f = |q-k| (1) or max(q-k, 0) (0)
  float softcap;         // > 0: s = softcap * tanh(s / softcap)
  const float* head_scale;  // [Hq] or null (not with softcap)
  float constant;
};

// Keys visible to query row q of batch b: [lo, hi], empty when lo > hi.
// kv_end = keys < kv_end exist (Lk, KVLenMask, QKVLengthMask); q_hi = rows
// < q_hi exist (Lq, QKVLengthMask).
__host__ __device__ inline void row_bounds(const ScoreMods& m, bool causal, int b, int kv_end,
                                           int q_hi, int q, int& lo, int& hi) {
  lo = 0;
  hi = kv_end - 1;
  if (q >= q_hi) {
    lo = 1;
    hi = 0;
    return;
  }
  if (causal) hi = min(hi, q + m.causal_shift);
  if (m.win_left != kNoBound) lo = max(lo, q - m.win_left);
  if (m.win_right != kNoBound) hi = min(hi, q + m.win_right);
  if (m.prefix) hi = min(hi, max(q, m.prefix[b] - 1));
  if (m.seqlen) {
    const int L = m.seqlen[b];
    if (q < L) {
      hi = min(hi, L - 1);
    } else {
      lo = max(lo, q);
      hi = min(hi, q);
    }
  }
}

// Query rows that see key k of batch b: [qlo, qhi] (the same relation as
// row_bounds, solved for q).
__host__ __device__ inline void key_bounds(const ScoreMods& m, bool causal, int b, int kv_end,
                                           int q_hi, int k, int& qlo, int& qhi) {
  qlo = 0;
  qhi = q_hi - 1;
  if (k >= kv_end) {
    qlo = 1;
    qhi = 0;
    return;
  }
  if (causal) qlo = max(qlo, k - m.causal_shift);
  if (m.win_right != kNoBound) qlo = max(qlo, k - m.win_right);
  if (m.win_left != kNoBound) qhi = min(qhi, k + m.win_left);
  if (m.prefix && k > m.prefix[b] - 1) qlo = max(qlo, k);
  if (m.seqlen) {
    const int L = m.seqlen[b];
    if (k < L) {
      qhi = min(qhi, L - 1);
    } else {
      qlo = max(qlo, k);
      qhi = min(qhi, k);
    }
  }
}

// Per-(head) constants of the score modifiers.
struct HeadMods {
  float slope;   // ALiBi slope of the head (0 without ALiBi)
  float hscale;  // per-head scale (1 without)
};

__device__ __forceinline__ HeadMods head_mods(const ScoreMods& m, int h) {
  HeadMods r;
  r.slope = m.alibi ? m.alibi[h] : 0.f;
  r.hscale = m.head_scale ? m.head_scale[h] : 1.f;
  return r;
}

// Modified score of s = sm_scale * q.k plus `add` (the dense bias), for
// query q and key k; g receives d(modified)/d(s).  Branch-free per score:
// an absent ALiBi term has slope 0, an absent head scale is 1; the soft cap
// is chosen per tile (SOFTCAP).
template <bool SOFTCAP>
__device__ __forceinline__ float modify_score(const ScoreMods& m, const HeadMods& hm, float s,
                                              float add, int q, int k, float& g) {
  if constexpr (SOFTCAP) {
    // tanh(x) = sign(x) * (1 - 2 / (1 + e^{2|x|})); e^{2|x|} -> inf gives 1.
    const float x = s * (1.f / m.softcap);
    const float e = __builtin_amdgcn_exp2f(2.f * 1.4426950408889634f * fabsf(x));
    const float t = copysignf(1.f - 2.f * __builtin_amdgcn_rcpf(1.f + e), x);
    s = m.softcap * t;
    g = 1.f - t * t;
  } else {
    s *= hm.hscale;
    g = hm.hscale;
  }
  const int d = q - k;
  const int f = m.alibi_sym ? abs(d) : max(d, 0);
  return fmaf(-hm.slope, (float)f, s) + add + m.constant;
}

}  // namespace pjx
