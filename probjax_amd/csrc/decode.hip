// Split-KV decode for gfx950: GQA decode (separate K/V, per-sequence lengths)
// and absorbed latent attention (MLA, K = V = one shared latent cache).
//
// Semantics: the split-KV forward of probjax
// (probjax/nn/pallas_kernels/kernels/attention_splitkv.py:43-250) -- every
// KV chunk yields a partial output and its softmax statistics, combined by an
// exact log-sum-exp merge -- extended with KVLenMask (keys >= L[b] masked,
// attention_mask_bias.py:1399-1532), whose reference semantics are those of
// xla_attention (kernels/attention_xla.py:339-429).  Query rows are packed per
// KV head: row = g*Lq + t for GQA (attention_splitkv.py:121-126) and
// row = t*H + h for MLA (heads folded, layers/latent_attention.py:458-469).
//
// Work decomposition (HBM-bound; compute is a few % of the MFMA rate):
//   * one workgroup per (batch, kv group, chunk of `chunk` keys); chunks past
//     the sequence's length exit at once, so only valid K/V is ever read;
//   * per 64-key tile, wave w loads keys [16w, 16w+16) directly from HBM as
//     the A operand of v_mfma_f32_16x16x32_bf16 (16-byte loads, 256 B per
//     row) and computes S^T (keys x 16 rows); the values are also scattered
//     into V^T in LDS (the shared latent is read once for both products);
//   * every wave reads the 64 x 16 score tile back from LDS, runs the online
//     softmax redundantly, and multiplies its own share of the output dims:
//     O^T[d][row] += V^T P^T, with V^T read as one 16-byte LDS load per step;
//   * the merge kernel combines the chunks of one (batch, group) exactly.
#include "pjx_common.h"
#include "pjx_internal.h"

namespace pjx {

constexpr int kDecThreads = 256;
constexpr int kTile = 64;       // keys per tile (16 per wave)
constexpr int kRows = 16;       // query rows per MFMA column block
constexpr int kSStride = kTile + 4;  // score tile row stride (floats)

struct DecodeArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* lengths;
  uint16_t* o;
  float* lse;
  float* ws_o;   // [B*G][nch][rows][dv] unnormalised partial outputs
  float* ws_ml;  // [B*G][nch][rows][2]  running max (log2 units), sum
  int B, Lq, Lk, Hq, G, rows;
  int fold;      // 1: row = t*H + h (MLA); 0: row = gi*Lq + t (GQA)
  int chunk, nch;
  int dv;        // output dims (<= D)
  float cx;      // sm_scale * log2(e)
};

__device__ __forceinline__ void row_to_head(const DecodeArgs& a, int g, int r, int& t, int& h) {
  if (a.fold) {
    t = r / a.Hq;
    h = r % a.Hq;
  } else {
    const int per = a.Hq / a.G;
    t = r % a.Lq;
    h = g * per + r / a.Lq;
  }
}

__device__ __forceinline__ int seq_len(const DecodeArgs& a, int b) {
  int L = a.Lk;
  if (a.lengths) L = min(L, max(a.lengths[b], 0));
  return L;
}

__device__ __forceinline__ float xor16_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Keeps the compiler from moving LDS accesses of one wave across this point;
// the LDS itself executes one wave's accesses in program order.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Writes the combined result of one work item: the final bf16 output and LSE
// when the item covers the whole sequence, else the unnormalised partial
// (O relative to max M, plus M and the sum) for the merge kernel.
__device__ __forceinline__ void emit_row_elem(const DecodeArgs& a, int b, int g, int r, int d,
                                              size_t part, bool final_out, float M, float Ls,
                                              float O) {
  if (final_out) {
    int t, h;
    row_to_head(a, g, r, t, h);
    const float out = Ls > 0.f ? O / Ls : 0.f;
    a.o[((size_t)(b * a.Lq + t) * a.Hq + h) * a.dv + d] = __builtin_bit_cast(uint16_t, (__bf16)out);
    if (a.lse && d == 0)
      a.lse[((size_t)b * a.Hq + h) * a.Lq + t] = Ls > 0.f ? (M + __log2f(Ls)) * kLn2 : INFINITY;
  } else {
    a.ws_o[(part * a.rows + r) * a.dv + d] = O;
    if (d == 0) {
      a.ws_ml[(part * a.rows + r) * 2] = M;
      a.ws_ml[(part * a.rows + r) * 2 + 1] = Ls;
    }
  }
}

// ---------------------------------------------------------------------------
// GQA split-KV decode.  One workgroup = one (chunk, batch, kv group) work
// item; its 4 waves split the chunk's keys into contiguous quarters and run
// independent online softmaxes (no block barrier inside the key loop), then
// combine their (max, sum, O) in LDS.  Per iteration a wave takes 32 keys:
//   * K rows are loaded straight into the A operand of
//     v_mfma_f32_16x16x32_bf16 (lane: key l%16, 16 bytes of dims), S^T = K Q^T
//     with the G*Lq query rows as the 16 MFMA columns;
//   * V rows are loaded 4 keys x 8 dims per lane, packed with v_perm into
//     [dim][key] order and written to a wave-private LDS slab, from which the
//     A operand of O^T += V^T P^T is two 8-byte reads;
//   * the next iteration's K and V loads are issued before this iteration's
//     softmax and P.V, so HBM traffic overlaps the arithmetic.
// Keys at or past the sequence length are never read.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256, 2) void gqa_decode_kernel(DecodeArgs a) {
  constexpr int KSTEPS = D / 32;  // 32-dim MFMA k-steps of Q.K
  constexpr int NDB = D / 16;     // 16-dim output blocks
  constexpr int DC = D / 8;       // 16-byte chunks per row
  constexpr int VU = D / 64;      // (4 keys x 8 dims) V units per lane per 32 keys
  constexpr int VTS = 36;         // V^T row stride (bf16): 32 keys + 4 pad
  static_assert(D % 64 == 0, "head dim");
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[4 * D * VTS];
  static_assert(4 * D * VTS * 2 >= 4 * 16 * D * 4 + 4 * 16 * 2 * 4, "combine scratch fits");

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c16 = lane & 15, q4 = lane >> 4;
  const int BG = a.B * a.G;
  const int chunk_id = blockIdx.x / BG;
  const int bg = blockIdx.x % BG;
  const int b = bg / a.G, g = bg % a.G;
  const int L = seq_len(a, b);
  const int c0 = chunk_id * a.chunk;
  if (c0 >= L) return;  // the whole workgroup: nothing past the length is read
  const int per_wave = a.chunk >> 2;
  const int w0 = c0 + w * per_wave;
  const int w1 = min(w0 + per_wave, L);

  bf16x8 qf[KSTEPS];
  {
    const bool rv = c16 < a.rows;
    int t = 0, h = 0;
    if (rv) row_to_head(a, g, c16, t, h);
    const uint16_t* qrow = a.q + ((size_t)(b * a.Lq + t) * a.Hq + h) * D;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      u32x4 r = {0u, 0u, 0u, 0u};
      if (rv) r = *(const u32x4*)(qrow + 32 * s + 8 * q4);
      qf[s] = as_bf16x8(r);
    }
  }
  const size_t kv_tok = (size_t)a.G * D;
  const uint16_t* Kb = a.k + ((size_t)b * a.Lk * a.G + g) * D;
  const uint16_t* Vb = a.v + ((size_t)b * a.Lk * a.G + g) * D;
  uint16_t* vl = vt_lds + w * D * VTS;

  f32x4 acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc[i] = f32x4{};
  float m_run = kMaxInit, l_run = 0.f;

  u32x4 kr[2][KSTEPS];
  u32x4 vr[VU][4];
  auto load_k = [&](int k0) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int key = k0 + 16 * kb + c16;
      const bool ok = key < w1;
      const uint16_t* p = Kb + (size_t)(ok ? key : 0) * kv_tok + 8 * q4;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        u32x4 r = {0u, 0u, 0u, 0u};
        if (ok) r = *(const u32x4*)(p + 32 * s);
        kr[kb][s] = r;
      }
    }
  };
  auto load_v = [&](int k0) {
#pragma unroll
    for (int i = 0; i < VU; ++i) {
      const int u = lane + 64 * i;
      const int dc = u % DC, kq = u / DC;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = k0 + 4 * kq + j;
        u32x4 r = {0u, 0u, 0u, 0u};
        if (key < w1) r = *(const u32x4*)(Vb + (size_t)key * kv_tok + 8 * dc);
        vr[i][j] = r;
      }
    }
  };
  auto store_vt = [&]() {
#pragma unroll
    for (int i = 0; i < VU; ++i) {
      const int u = lane + 64 * i;
      const int dc = u % DC, kq = u / DC;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int dw = e >> 1;
        u32x2 pk;
        if (e & 1) {
          pk[0] = pack_hi_halves(vr[i][0][dw], vr[i][1][dw]);
          pk[1] = pack_hi_halves(vr[i][2][dw], vr[i][3][dw]);
        } else {
          pk[0] = pack_lo_halves(vr[i][0][dw], vr[i][1][dw]);
          pk[1] = pack_lo_halves(vr[i][2][dw], vr[i][3][dw]);
        }
        *(u32x2*)(vl + (8 * dc + e) * VTS + 4 * kq) = pk;
      }
    }
  };

  if (w0 < w1) {
    load_k(w0);
    load_v(w0);
  }
  for (int k0 = w0; k0 < w1; k0 += 32) {
    const int kn = k0 + 32;
    store_vt();
    if (kn < w1) load_v(kn);
    // S^T for keys k0 + 16*kb + 4*q4 + r (register r), query row c16.
    f32x4 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f32x4{};
#pragma unroll
      for (int st = 0; st < KSTEPS; ++st) s[kb] = mfma16x16x32(as_bf16x8(kr[kb][st]), qf[st], s[kb]);
    }
    if (kn < w1) load_k(kn);
    if (kn > w1) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (k0 + 16 * kb + 4 * q4 + r >= w1) s[kb][r] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = xor32_max(xor16_max(mx));
    const float m_new = fmaxf(m_run, mx * a.cx);
    const float corr = fast_exp2(m_run - m_new);
    m_run = m_new;
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = fast_exp2(fmaf(s[kb][r], a.cx, -m_new));
        rs += p;
        s[kb][r] = p;
      }
    l_run = fmaf(l_run, corr, rs);
    // P^T as the B operand: slot j < 4 <-> key 4*q4 + j, slot j >= 4 <-> key 16 + 4*q4 + j - 4.
    u32x4 pk;
    pk[0] = pack_bf16x2(s[0][0], s[0][1]);
    pk[1] = pack_bf16x2(s[0][2], s[0][3]);
    pk[2] = pack_bf16x2(s[1][0], s[1][1]);
    pk[3] = pack_bf16x2(s[1][2], s[1][3]);
    const bf16x8 pf = as_bf16x8(pk);
    wave_lds_sync();
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const uint16_t* vp = vl + (16 * db + c16) * VTS + 4 * q4;
      const u32x2 lo = *(const u32x2*)vp;
      const u32x2 hi = *(const u32x2*)(vp + 16);
      const u32x4 av = {lo[0], lo[1], hi[0], hi[1]};
      acc[db] *= corr;
      acc[db] = mfma16x16x32(as_bf16x8(av), pf, acc[db]);
    }
    wave_lds_sync();
  }

  // ---- combine the 4 waves of this work item ----
  l_run = xor32_sum(xor16_sum(l_run));
  __syncthreads();  // every wave is done with its V^T slab
  float* red_o = (float*)vt_lds;           // [4][16 rows][D]
  float* red_ml = red_o + 4 * 16 * D;      // [4][16 rows][2]
#pragma unroll
  for (int db = 0; db < NDB; ++db)
    *(f32x4*)(red_o + (w * 16 + c16) * D + 16 * db + 4 * q4) = acc[db];
  if (q4 == 0) {
    red_ml[(w * 16 + c16) * 2] = m_run;
    red_ml[(w * 16 + c16) * 2 + 1] = l_run;
  }
  __syncthreads();
  const bool final_out = c0 == 0 && L <= a.chunk;
  const size_t part = (size_t)bg * a.nch + chunk_id;
  for (int e = tid; e < a.rows * D; e += 256) {
    const int r = e / D, d = e % D;
    float M = kMaxInit;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, red_ml[(ww * 16 + r) * 2]);
    float Ls = 0.f, O = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float wt = fast_exp2(red_ml[(ww * 16 + r) * 2] - M);
      Ls = fmaf(wt, red_ml[(ww * 16 + r) * 2 + 1], Ls);
      O = fmaf(wt, red_o[(ww * 16 + r) * D + d], O);
    }
    emit_row_elem(a, b, g, r, d, part, final_out, M, Ls, O);
  }
}

// D: q.k dims; NDT: 16-wide output-dim tiles per wave (DV = 64*NDT);
// SHARED: V is the first DV dims of K (absorbed MLA).
template <int D, int NDT, bool SHARED>
__global__ __launch_bounds__(kDecThreads) void decode_chunk_kernel(DecodeArgs a) {
  constexpr int DV = 64 * NDT;
  constexpr int KSTEPS = D / 32;
  constexpr int VT = kTile + 8;  // V^T row stride (bf16): 144 B rows keep b128 reads aligned
  static_assert(DV <= D || !SHARED, "shared V must be a prefix of K");
  static_assert(D % 32 == 0, "head dim");

  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[DV * VT];
  __shared__ __attribute__((aligned(16))) float s_lds[kRows * kSStride];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c16 = lane & 15, q4 = lane >> 4;
  const int chunk_id = blockIdx.x % a.nch;
  const int bg = blockIdx.x / a.nch;
  const int b = bg / a.G, g = bg % a.G;
  const int L = seq_len(a, b);
  const int c0 = chunk_id * a.chunk;
  if (c0 >= L) return;  // whole workgroup exits: nothing past the length is read
  const int c1 = min(c0 + a.chunk, L);

  // Q as the B operand: lane holds row c16, dims 32*s + 8*q4 + [0,8).
  bf16x8 qf[KSTEPS];
  {
    const bool rv = c16 < a.rows;
    int t = 0, h = 0;
    if (rv) row_to_head(a, g, c16, t, h);
    const uint16_t* qrow = a.q + ((size_t)(b * a.Lq + t) * a.Hq + h) * D;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      u32x4 r = {0u, 0u, 0u, 0u};
      if (rv) r = *(const u32x4*)(qrow + 32 * s + 8 * q4);
      qf[s] = as_bf16x8(r);
    }
  }
  const size_t kv_tok = (size_t)a.G * D;
  const uint16_t* Kb = a.k + ((size_t)b * a.Lk * a.G + g) * D;
  const uint16_t* Vb = SHARED ? Kb : a.v + ((size_t)b * a.Lk * a.G + g) * D;

  f32x4 acc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = f32x4{};
  float m_run = kMaxInit, l_run = 0.f;

  for (int k0 = c0; k0 < c1; k0 += kTile) {
    // ---- phase 1: S^T for keys [k0 + 16w, +16), V^T into LDS ----
    const int key = k0 + 16 * w + c16;
    const bool kin = key < c1;
    const uint16_t* krow = Kb + (size_t)(kin ? key : 0) * kv_tok;
    u32x4 kf[KSTEPS];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      u32x4 r = {0u, 0u, 0u, 0u};
      if (kin) r = *(const u32x4*)(krow + 32 * s + 8 * q4);
      kf[s] = r;
    }
    u32x4 vf[SHARED ? 1 : DV / 32];
    if constexpr (!SHARED) {
      const uint16_t* vrow = Vb + (size_t)(kin ? key : 0) * kv_tok;
#pragma unroll
      for (int s = 0; s < DV / 32; ++s) {
        u32x4 r = {0u, 0u, 0u, 0u};
        if (kin) r = *(const u32x4*)(vrow + 32 * s + 8 * q4);
        vf[s] = r;
      }
    }
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) sacc = mfma16x16x32(as_bf16x8(kf[s]), qf[s], sacc);
    // C layout: lane holds row c16, keys 16w + 4*q4 + r.
    *(f32x4*)(&s_lds[c16 * kSStride + 16 * w + 4 * q4]) = sacc;
    // V^T[d][key - k0]
    {
      const int kc = 16 * w + c16;
#pragma unroll
      for (int s = 0; s < DV / 32; ++s) {
        const u32x4 src = SHARED ? kf[s] : vf[SHARED ? 0 : s];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d = 32 * s + 8 * q4 + 2 * j;
          vt_lds[d * VT + kc] = (uint16_t)(src[j] & 0xffffu);
          vt_lds[(d + 1) * VT + kc] = (uint16_t)(src[j] >> 16);
        }
      }
    }
    __syncthreads();

    // ---- phase 2: softmax over the 64-key tile, then O^T += V^T P^T ----
    float p[2][8];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const f32x4 lo = *(const f32x4*)(&s_lds[c16 * kSStride + 32 * c + 8 * q4]);
      const f32x4 hi = *(const f32x4*)(&s_lds[c16 * kSStride + 32 * c + 8 * q4 + 4]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p[c][j] = lo[j];
        p[c][4 + j] = hi[j];
      }
    }
    if (k0 + kTile > c1) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (k0 + 32 * c + 8 * q4 + j >= c1) p[c][j] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, p[c][j]);
    mx = xor16_max(mx);
    mx = xor32_max(mx);
    const float m_new = fmaxf(m_run, mx * a.cx);
    const float corr = fast_exp2(m_run - m_new);
    m_run = m_new;
    float rs = 0.f;
    bf16x8 pf[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      u32x4 pk;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e0 = fast_exp2(fmaf(p[c][2 * j], a.cx, -m_new));
        const float e1 = fast_exp2(fmaf(p[c][2 * j + 1], a.cx, -m_new));
        rs += e0 + e1;
        pk[j] = pack_bf16x2(e0, e1);
      }
      pf[c] = as_bf16x8(pk);
    }
    l_run = fmaf(l_run, corr, rs);
#pragma unroll
    for (int i = 0; i < NDT; ++i) {
      acc[i] *= corr;
      const int dt = w * NDT + i;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const u32x4 av = *(const u32x4*)(&vt_lds[(dt * 16 + c16) * VT + 32 * c + 8 * q4]);
        acc[i] = mfma16x16x32(as_bf16x8(av), pf[c], acc[i]);
      }
    }
    __syncthreads();
  }

  // ---- this chunk's result: final output if it covers the sequence ----
  l_run = xor16_sum(l_run);
  l_run = xor32_sum(l_run);
  const size_t part = (size_t)bg * a.nch + chunk_id;
  const bool final_out = c0 == 0 && L <= a.chunk;
  if (c16 < a.rows) {
#pragma unroll
    for (int i = 0; i < NDT; ++i) {
      const int d0 = (w * NDT + i) * 16 + 4 * q4;
      if (d0 < a.dv) {
#pragma unroll
        for (int j = 0; j < 4; ++j) emit_row_elem(a, b, g, c16, d0 + j, part, final_out, m_run, l_run, acc[i][j]);
      }
    }
  }
}

// Exact merge of the chunk partials of one (batch, group, query row):
// M = max_c m_c, O = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c
// (attention_splitkv.py:236-245, with unnormalised partials).  Sequences that
// fit one chunk were finished by the chunk kernel; empty sequences (length 0,
// no chunk ran) get a zero output and LSE = +inf (attention_xla.py:417-420).
__global__ __launch_bounds__(128) void decode_merge_kernel(DecodeArgs a) {
  constexpr int kMaxBatch = 512;  // chunk weights staged in LDS per pass
  __shared__ float wts[kMaxBatch];
  __shared__ float red[2][4];
  const int bg = blockIdx.x / a.rows;
  const int r = blockIdx.x % a.rows;
  const int b = bg / a.G, g = bg % a.G;
  const int L = seq_len(a, b);
  const int n = (L + a.chunk - 1) / a.chunk;
  if (n == 1) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const size_t base = (size_t)bg * a.nch;
  const float* ml = a.ws_ml + (base * a.rows + r) * 2;  // chunk c at ml[c * rows * 2]
  const size_t ml_stride = (size_t)a.rows * 2;
  // Global max of the chunk maxima.
  float M = kMaxInit;
  for (int c = tid; c < n; c += 128) M = fmaxf(M, ml[c * ml_stride]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
  if (lane == 0) red[0][w] = M;
  __syncthreads();
  M = fmaxf(red[0][0], red[0][1]);
  int t, h;
  row_to_head(a, g, r, t, h);
  uint16_t* orow = a.o + ((size_t)(b * a.Lq + t) * a.Hq + h) * a.dv;
  const float* po = a.ws_o + (base * a.rows + r) * a.dv;  // chunk c at po[c * rows * dv]
  const size_t o_stride = (size_t)a.rows * a.dv;
  float num[5] = {0.f, 0.f, 0.f, 0.f, 0.f};  // dv <= 640 over 128 threads
  float den = 0.f;
  for (int cb = 0; cb < n; cb += kMaxBatch) {
    const int cn = min(kMaxBatch, n - cb);
    __syncthreads();
    for (int c = tid; c < cn; c += 128) {
      const float wt = fast_exp2(ml[(size_t)(cb + c) * ml_stride] - M);
      wts[c] = wt;
      den = fmaf(wt, ml[(size_t)(cb + c) * ml_stride + 1], den);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      const int d = tid + 128 * i;
      if (d < a.dv) {
        const float* p = po + (size_t)cb * o_stride + d;
        float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
        int c = 0;
        for (; c + 4 <= cn; c += 4) {
          acc0 = fmaf(wts[c], p[(size_t)c * o_stride], acc0);
          acc1 = fmaf(wts[c + 1], p[(size_t)(c + 1) * o_stride], acc1);
          acc2 = fmaf(wts[c + 2], p[(size_t)(c + 2) * o_stride], acc2);
          acc3 = fmaf(wts[c + 3], p[(size_t)(c + 3) * o_stride], acc3);
        }
        for (; c < cn; ++c) acc0 = fmaf(wts[c], p[(size_t)c * o_stride], acc0);
        num[i] += (acc0 + acc1) + (acc2 + acc3);
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o);
  if (lane == 0) red[1][w] = den;
  __syncthreads();
  den = red[1][0] + red[1][1];
  const float inv = den > 0.f ? 1.f / den : 0.f;
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int d = tid + 128 * i;
    if (d < a.dv) orow[d] = __builtin_bit_cast(uint16_t, (__bf16)(num[i] * inv));
  }
  if (a.lse && tid == 0)
    a.lse[((size_t)b * a.Hq + h) * a.Lq + t] = den > 0.f ? (M + __log2f(den)) * kLn2 : INFINITY;
}

// Keys per work item when the caller passes chunk = 0: the smallest power of
// two in [128, 2048] that leaves at most `items` (chunk, batch, group) work
// items at full capacity.  Longer items amortise the per-item start-up (Q
// fragments, the cross-wave combine, partial writes); the item target keeps
// short batches spread over every CU.  Measured on MI355X: the GQA decode is
// fastest with ~512 items at capacity (2048-key chunks for 32 x 8 x 8192), the
// latent decode with ~256 (256-key chunks for 16 x 4096).
constexpr int64_t kGqaItems = 512;
constexpr int64_t kMlaItems = 256;

static int64_t auto_chunk(int64_t batch, int64_t groups, int64_t kv_len, int64_t items) {
  const int64_t work = batch * groups * std::max<int64_t>(kv_len, 1);
  int64_t c = 128;
  while (c < 2048 && work / c > items) c *= 2;
  return c;
}

static size_t ws_size(int64_t batch, int64_t groups, int64_t rows, int64_t kv_len,
                      int64_t v_dim, int64_t chunk) {
  // chunk = 0: size for the smaller of the two automatic choices, which is
  // enough for either decode entry point.
  if (chunk <= 0)
    chunk = std::min(auto_chunk(batch, groups, kv_len, kGqaItems), auto_chunk(batch, groups, kv_len, kMlaItems));
  const int64_t nch = (kv_len + chunk - 1) / chunk;
  const int64_t parts = batch * groups * std::max<int64_t>(nch, 1) * rows;
  return (size_t)(parts * v_dim + parts * 2) * sizeof(float);
}

template <typename K>
static int run_decode(K kernel, DecodeArgs& a, void* workspace, size_t ws_bytes,
                      hipStream_t stream, const char* name) {
  const size_t need = ws_size(a.B, a.G, a.rows, a.Lk, a.dv, a.chunk);
  if (!workspace || ws_bytes < need) return fail(PJX_ERR_WORKSPACE, "decode: workspace missing or too small");
  const size_t parts = (size_t)a.B * a.G * a.nch * a.rows;
  a.ws_o = (float*)workspace;
  a.ws_ml = a.ws_o + parts * a.dv;
  const long blocks = (long)a.B * a.G * a.nch;
  if (blocks > 0x7fffffffL || (long)a.B * a.G * a.rows > 0x7fffffffL)
    return fail(PJX_ERR_INVALID, "decode: grid too large");
  hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(kDecThreads), 0, stream, a);
  int rc = check_launch(name);
  if (rc) return rc;
  hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)(a.B * a.G * a.rows)), dim3(128), 0, stream, a);
  return check_launch(name);
}

}  // namespace pjx

using namespace pjx;

extern "C" size_t pjx_decode_workspace_size(int64_t batch, int64_t groups, int64_t rows,
                                            int64_t kv_len, int64_t v_dim, int64_t chunk) {
  return ws_size(batch, groups, rows, kv_len, v_dim, chunk);
}

extern "C" int pjx_splitkv_decode(int dtype, const void* q, const void* k, const void* v,
                                  const int32_t* kv_lengths, void* o, float* lse,
                                  void* workspace, size_t workspace_bytes, int64_t batch,
                                  int64_t q_len, int64_t kv_len, int64_t q_heads,
                                  int64_t kv_heads, int64_t head_dim, float sm_scale,
                                  int64_t chunk, void* stream) {
  clear_error();
  if (dtype != PJX_DTYPE_BF16) return fail(PJX_ERR_INVALID, "pjx_splitkv_decode: only bf16 is supported");
  if (!q || !k || !v || !o) return fail(PJX_ERR_INVALID, "pjx_splitkv_decode: null pointer");
  if (batch < 0 || q_len <= 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads)
    return fail(PJX_ERR_INVALID, "pjx_splitkv_decode: bad sizes");
  if (head_dim != 128 && head_dim != 64) return fail(PJX_ERR_INVALID, "pjx_splitkv_decode: head_dim must be 64 or 128");
  const int64_t rows = (q_heads / kv_heads) * q_len;
  if (rows > kRows) return fail(PJX_ERR_INVALID, "pjx_splitkv_decode: (Hq/Hkv)*Lq must be <= 16");
  if (!(sm_scale > 0.f)) return fail(PJX_ERR_INVALID, "pjx_splitkv_decode: sm_scale must be > 0");
  if (chunk == 0) chunk = auto_chunk(batch, kv_heads, kv_len, kGqaItems);
  if (chunk < 128 || chunk % 128) return fail(PJX_ERR_INVALID, "pjx_splitkv_decode: chunk must be a positive multiple of 128");
  if (kv_len > (1 << 30) || batch * kv_len * kv_heads * head_dim > ((int64_t)1 << 40))
    return fail(PJX_ERR_INVALID, "pjx_splitkv_decode: sizes out of range");
  if (batch == 0) return PJX_OK;
  DecodeArgs a = {};
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
  a.lengths = kv_lengths; a.o = (uint16_t*)o; a.lse = lse;
  a.B = (int)batch; a.Lq = (int)q_len; a.Lk = (int)kv_len; a.Hq = (int)q_heads; a.G = (int)kv_heads;
  a.rows = (int)rows; a.fold = 0; a.chunk = (int)chunk;
  a.nch = (int)std::max<int64_t>((kv_len + chunk - 1) / chunk, 1);
  a.dv = (int)head_dim; a.cx = sm_scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128) return run_decode(gqa_decode_kernel<128>, a, workspace, workspace_bytes, s, "pjx_splitkv_decode");
  return run_decode(gqa_decode_kernel<64>, a, workspace, workspace_bytes, s, "pjx_splitkv_decode");
}

extern "C" int pjx_mla_decode(int dtype, const void* q, const void* cache,
                              const int32_t* kv_lengths, void* o, float* lse, void* workspace,
                              size_t workspace_bytes, int64_t batch, int64_t q_len,
                              int64_t heads, int64_t kv_len, int64_t rank, int64_t v_dim,
                              float sm_scale, int64_t chunk, void* stream) {
  clear_error();
  if (dtype != PJX_DTYPE_BF16) return fail(PJX_ERR_INVALID, "pjx_mla_decode: only bf16 is supported");
  if (!q || !cache || !o) return fail(PJX_ERR_INVALID, "pjx_mla_decode: null pointer");
  if (batch < 0 || q_len <= 0 || heads <= 0 || kv_len < 0) return fail(PJX_ERR_INVALID, "pjx_mla_decode: bad sizes");
  if (q_len * heads > kRows) return fail(PJX_ERR_INVALID, "pjx_mla_decode: Lq*H must be <= 16");
  if (!(sm_scale > 0.f)) return fail(PJX_ERR_INVALID, "pjx_mla_decode: sm_scale must be > 0");
  if (chunk == 0) chunk = auto_chunk(batch, 1, kv_len, kMlaItems);
  if (chunk < kTile || chunk % kTile) return fail(PJX_ERR_INVALID, "pjx_mla_decode: chunk must be a positive multiple of 64");
  if (kv_len > (1 << 30) || batch * kv_len * rank > ((int64_t)1 << 40))
    return fail(PJX_ERR_INVALID, "pjx_mla_decode: sizes out of range");
  DecodeArgs a = {};
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)cache; a.v = (const uint16_t*)cache;
  a.lengths = kv_lengths; a.o = (uint16_t*)o; a.lse = lse;
  a.B = (int)batch; a.Lq = (int)q_len; a.Lk = (int)kv_len; a.Hq = (int)heads; a.G = 1;
  a.rows = (int)(q_len * heads); a.fold = 1; a.chunk = (int)chunk;
  a.nch = (int)std::max<int64_t>((kv_len + chunk - 1) / chunk, 1);
  a.dv = (int)v_dim; a.cx = sm_scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  if (batch == 0) return PJX_OK;
  if (rank == 576 && v_dim == 512) return run_decode(decode_chunk_kernel<576, 8, true>, a, workspace, workspace_bytes, s, "pjx_mla_decode");
  if (rank == 576 && v_dim == 576) return run_decode(decode_chunk_kernel<576, 9, true>, a, workspace, workspace_bytes, s, "pjx_mla_decode");
  if (rank == 512 && v_dim == 512) return run_decode(decode_chunk_kernel<512, 8, true>, a, workspace, workspace_bytes, s, "pjx_mla_decode");
  if (rank == 128 && v_dim == 128) return run_decode(decode_chunk_kernel<128, 2, true>, a, workspace, workspace_bytes, s, "pjx_mla_decode");
  return fail(PJX_ERR_INVALID, "pjx_mla_decode: supported (rank, v_dim): (576,512), (576,576), (512,512), (128,128)");
}
