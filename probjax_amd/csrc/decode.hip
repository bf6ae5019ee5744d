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
//   * GQA (gqa_decode_kernel): the 4 waves split the chunk's keys, load K rows
//     straight into MFMA operands and V through a per-wave LDS slab, and
//     combine their (max, sum, O) in LDS at the end;
//   * latent (mla_decode_kernel): 64-key tiles of the shared latent go
//     HBM -> LDS; each wave forms S^T for 16 keys, the 64 x 16 score tile is
//     shared through LDS, every wave runs the same online softmax over it and
//     multiplies its own quarter of the output dims, so no combine is needed;
//   * the merge kernel combines the chunks of one (batch, group) exactly.
// Inputs are bf16 or fp16 (the kernels are templated on the 16-bit format;
// the v_mfma_*_bf16 named here are v_mfma_*_f16 for fp16) or fp32 (GQA only).
#include <stdio.h>
#include <stdlib.h>

#include <atomic>

#include "pjx_common.h"
#include "pjx_internal.h"

namespace pjx {

constexpr int kDecThreads = 256;
constexpr int kTile = 64;       // keys per latent tile (16 per wave)
constexpr int kRows = 16;       // query rows per MFMA column block

struct DecodeArgs {
  const uint16_t* q;   // bf16 / fp16 (fp32 decode: the same pointers hold floats)
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* lengths;
  uint16_t* o;         // 16-bit output (bf16, or fp16 when f16), or null with o32
  float* o32;          // fp32 output of the fp32 decode, else null
  int f16;             // 16-bit inputs and output are fp16 (else bf16)
  float* lse;
  float* ws_o;   // [B*G][nch][rows][dv] unnormalised partial outputs
  float* ws_ml;  // [B*G][nch][rows][2]  running max (log2 units), sum
  int B, Lq, Lk, Hq, G, rows;
  int fold;      // 1: row = t*H + h (MLA); 0: row = gi*Lq + t (GQA)
  int chunk, nch;
  int dv;        // output dims
  float cx;      // sm_scale * log2(e)
  // Query rows per row group: the rows of a KV head are split into groups of
  // `rpg` (16 per MFMA column block of the kernel), one per blockIdx.y; each
  // group's workgroups stream the same keys.
  int rpg;
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


// Keeps the compiler from moving LDS accesses of one wave across this point;
// the LDS itself executes one wave's accesses in program order.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Writes the combined result of one work item: the final 16-bit output and LSE
// when the item covers the whole sequence, else the unnormalised partial
// (O relative to max M, plus M and the sum) for the merge kernel.
__device__ __forceinline__ void emit_row_elem(const DecodeArgs& a, int b, int g, int r, int d,
                                              size_t part, bool final_out, float M, float Ls,
                                              float O) {
  if (final_out) {
    int t, h;
    row_to_head(a, g, r, t, h);
    const float out = Ls > 0.f ? O / Ls : 0.f;
    const size_t oi = ((size_t)(b * a.Lq + t) * a.Hq + h) * a.dv + d;
    if (a.o32)
      a.o32[oi] = out;
    else
      a.o[oi] = a.f16 ? F16Fmt::bits(out) : Bf16Fmt::bits(out);
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

// Work item of a decode workgroup: (batch b, kv group g, chunk chunk_id).
// The hardware starts workgroups in index order as slots free up, so the
// index order is the schedule.  With per-sequence lengths (B <=
// kSchedMaxBatch) the items run longest first: every full chunk (sequence by
// sequence, or chunk-major where every sequence has as many), then each
// sequence's partial last chunk in decreasing size, then
// the empty items, which exit at once.  The plain chunk-major order scatters
// the partial chunks through the grid and leaves a tail of full chunks that
// start late.  Every thread calls this (it holds two barriers); L receives
// the sequence's clamped length; false: the item has no keys.
constexpr int kSchedMaxBatch = 256;
static_assert(kSchedMaxBatch <= kDecThreads, "one length per thread");
__device__ bool decode_item(const DecodeArgs& a, int* sched, int& b, int& g, int& chunk_id, int& L) {
  if (!a.lengths || a.B > kSchedMaxBatch) {
    const int BG = a.B * a.G;
    chunk_id = blockIdx.x / BG;
    const int bg = blockIdx.x % BG;
    b = bg / a.G;
    g = bg % a.G;
    L = seq_len(a, b);
    return chunk_id * a.chunk < L;
  }
  const int q = blockIdx.x / a.G, t = threadIdx.x;
  g = blockIdx.x % a.G;
  int* nfs = sched + 4;                 // full chunks per sequence
  int* rms = nfs + kSchedMaxBatch;      // keys of the partial last chunk
  int Lt = 0, nf = 0, rt = 0;
  if (t < a.B) {
    Lt = seq_len(a, t);
    nf = Lt / a.chunk;
    rt = Lt - nf * a.chunk;
    nfs[t] = nf;
    rms[t] = rt;
  }
  if (t == 0) sched[0] = -1;
  __syncthreads();
  if (t < a.B) {
    // sequence t: its full chunks are rows [pre, pre + nf) of the full part;
    // its partial chunk (rt > 0) has the rank of rt among the partial chunks
    // (ties by sequence index)
    int pre = 0, full = 0, rank = 0, nf_min = nf, nf_max = nf;
#pragma unroll 8
    for (int u = 0; u < a.B; ++u) {
      const int nu = nfs[u], ru = rms[u];
      full += nu;
      pre += u < t ? nu : 0;
      nf_min = min(nf_min, nu);
      nf_max = max(nf_max, nu);
      rank += (ru > 0 && (ru > rt || (ru == rt && u < t))) ? 1 : 0;
    }
    int c = -1;
    if (nf_min == nf_max) {
      // as many full chunks in every sequence: chunk-major, as without lengths
      if (q < full && q % a.B == t) c = q / a.B;
    } else if (q >= pre && q < pre + nf) {
      c = q - pre;
    }
    if (rt > 0 && q >= full && q - full == rank) c = nf;
    if (c >= 0) {
      sched[0] = t;
      sched[1] = c;
      sched[2] = Lt;
    }
  }
  __syncthreads();
  b = sched[0];
  chunk_id = sched[1];
  L = sched[2];
  if (b < 0) {
    b = 0;
    L = 0;
    return false;
  }
  return true;
}

// emit_row_elem for 4 consecutive dims d..d+3 (d a multiple of 4).
__device__ __forceinline__ void emit_row_quad(const DecodeArgs& a, int b, int g, int r, int d,
                                              size_t part, bool final_out, float M, float Ls,
                                              f32x4 O) {
  if (final_out) {
    int t, h;
    row_to_head(a, g, r, t, h);
    const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
    const size_t oi = ((size_t)(b * a.Lq + t) * a.Hq + h) * a.dv + d;
    if (a.o32) {
      *(f32x4*)(a.o32 + oi) = O * inv;
    } else {
      const u32x2 pk = a.f16 ? u32x2{F16Fmt::pack2(O[0] * inv, O[1] * inv), F16Fmt::pack2(O[2] * inv, O[3] * inv)}
                             : u32x2{Bf16Fmt::pack2(O[0] * inv, O[1] * inv), Bf16Fmt::pack2(O[2] * inv, O[3] * inv)};
      *(u32x2*)(a.o + oi) = pk;
    }
    if (a.lse && d == 0)
      a.lse[((size_t)b * a.Hq + h) * a.Lq + t] = Ls > 0.f ? (M + __log2f(Ls)) * kLn2 : INFINITY;
  } else {
    *(f32x4*)(a.ws_o + (part * a.rows + r) * a.dv + d) = O;
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
// combine their (max, sum, O) in LDS.  The rows = (Hq/Hkv)*Lq query rows of
// the KV head are NRB blocks of 16 MFMA columns (up to 64 rows, the
// reference's largest packed tile, attention_splitkv.py:155-170).  Per
// iteration a wave takes 32 keys:
//   * K rows are loaded straight into the A operand of
//     v_mfma_f32_16x16x32_bf16 (lane: key l%16, 16 bytes of dims), S^T = K Q^T
//     for each row block;
//   * V rows are loaded 4 keys x 8 dims per lane, packed with v_perm into
//     [dim][key] order and written to a wave-private LDS slab, from which the
//     A operand of O^T += V^T P^T is two 8-byte reads, shared by the row
//     blocks;
//   * the next iteration's K and V loads are issued before this iteration's
//     softmax and P.V, so HBM traffic overlaps the arithmetic.
// Keys at or past the sequence length are never read.
// ---------------------------------------------------------------------------

// Combines the 4 waves' (max, sum, O^T) of row block rb through LDS scratch
// red (>= 4 x 16 x D floats + 4 x 16 x 2) and emits rows row0 + 16rb .. of the
// item (D = the output dims).  acc[i] holds O^T[dim 16i + 4*q4 + r][row
// row0 + 16rb + c16].
template <int D>
__device__ __forceinline__ void combine_rows(const DecodeArgs& a, float* red, const f32x4* acc,
                                             float m_run, float l_run, int row0, int rb, int b, int g,
                                             size_t part, bool final_out) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c16 = lane & 15, q4 = lane >> 4;
  float* red_o = red;                  // [4][16 rows][D]
  float* red_ml = red_o + 4 * 16 * D;  // [4][16 rows][2]
  __syncthreads();  // the scratch is free (every wave is done with it)
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
    *(f32x4*)(red_o + (w * 16 + c16) * D + 16 * db + 4 * q4) = acc[db];
  if (q4 == 0) {
    red_ml[(w * 16 + c16) * 2] = m_run;
    red_ml[(w * 16 + c16) * 2 + 1] = l_run;
  }
  __syncthreads();
  const int nr = min(16, a.rows - row0 - 16 * rb);
  for (int e = tid; e < nr * D; e += 256) {
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
    emit_row_elem(a, b, g, row0 + 16 * rb + r, d, part, final_out, M, Ls, O);
  }
}

// Two workgroups per CU where the registers allow it: 16- or 32-row groups at
// head dims up to 128.
template <int D, int DV, int NRB>
constexpr int decode_occupancy() { return (NRB == 4 || D > 128 || DV > 128) ? 1 : 2; }

template <typename E, int D, int DV, int NRB, bool STREAM>
__global__ __launch_bounds__(256, (decode_occupancy<D, DV, NRB>())) void gqa_decode_kernel(DecodeArgs a) {
  constexpr int KSTEPS = D / 32;  // 32-dim MFMA k-steps of Q.K
  constexpr int NDB = DV / 16;    // 16-dim output blocks
  constexpr int DC = DV / 8;      // 16-byte chunks per V row
  constexpr int VU = DV / 64;     // (4 keys x 8 dims) V units per lane per 32 keys
  constexpr int CR = D / 8;       // 16-byte chunks per K row
  constexpr int KLD = D / 16;     // K chunks per lane per 32-key step (32 * CR / 64 = 2 * KSTEPS)
  static_assert(D % 64 == 0 && DV % 64 == 0, "head dims");
  // Each wave's V^T tile: DV rows (output dims) of the step's 32 keys, 64
  // bytes each, 4 rows to a 256-byte bank line (see vt_at); the same memory
  // then holds the 4 waves' partial rows for the combine.
  constexpr int VT_B = 4 * DV * 64, COMB_B = 4 * 16 * DV * 4 + 4 * 16 * 2 * 4;
  __shared__ __attribute__((aligned(256))) uint16_t vt_lds[(VT_B > COMB_B ? VT_B : COMB_B) / 2];
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[STREAM ? 4 * 32 * D : 8];  // per wave: 32 key rows
  // STREAM: chunk swizzle of K row r in the wave's K slab, a bijection of the
  // row's 16-byte chunks that sends the same chunk of 16 consecutive rows to
  // 16 different bank groups (rows of 128, 256 or 512 bytes)
  auto kswz = [](int r) { return CR >= 16 ? (r & 15) : ((r >> 1) & (CR - 1)); };
  // STREAM: K/V are read once per call, past what the 256 MB MALL holds, with
  // non-temporal loads (measured on this layout: ~7.0 TB/s with full 128-byte
  // lines, against ~5.9 TB/s for ordinary loads)
  auto ld16 = [](const uint16_t* p) -> u32x4 {
    if constexpr (STREAM) return __builtin_nontemporal_load((const u32x4*)p);
    else return *(const u32x4*)p;
  };

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c16 = lane & 15, q4 = lane >> 4;
  __shared__ int sched[4 + 2 * kSchedMaxBatch];
  int b, g, chunk_id, L;
  if (!decode_item(a, sched, b, g, chunk_id, L)) return;  // nothing past the length is read
  const int bg = b * a.G + g;
  const int c0 = chunk_id * a.chunk;
  // the item's keys split evenly over the 4 waves (32-key steps), so a
  // partial chunk takes a quarter of its length, not up to a full quarter
  // chunk on one wave
  const int per_wave = ((min(L - c0, a.chunk) + 127) >> 7) << 5;
  const int w0 = c0 + w * per_wave;
  const int w1 = min(w0 + per_wave, L);

  const int row0 = blockIdx.y * 16 * NRB;  // this row group's first row
  typename E::v8 qf[NRB][KSTEPS];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    const int row = row0 + 16 * rb + c16;
    const bool rv = row < a.rows;
    int t = 0, h = 0;
    if (rv) row_to_head(a, g, row, t, h);
    const uint16_t* qrow = a.q + ((size_t)(b * a.Lq + t) * a.Hq + h) * D;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      u32x4 r = {0u, 0u, 0u, 0u};
      if (rv) r = *(const u32x4*)(qrow + 32 * s + 8 * q4);
      qf[rb][s] = E::as8(r);
    }
  }
  const size_t k_tok = (size_t)a.G * D, v_tok = (size_t)a.G * DV;
  const uint16_t* Kb = a.k + ((size_t)b * a.Lk * a.G + g) * D;
  const uint16_t* Vb = a.v + ((size_t)b * a.Lk * a.G + g) * DV;
  uint16_t* vl = vt_lds + w * DV * 32;
  // Element offset of 8-byte unit u (keys 4u .. 4u+3) of V^T row r.  The 32
  // units of a 256-byte line (rows 4L .. 4L+3) are XOR-swizzled by F(L) so
  // that both access patterns are free of bank conflicts: the writes of 16
  // lanes (one LDS cycle for ds_write_b64) put one unit of rows 8*dc + e,
  // dc = 0..15, in 16 different lines, whose F values all differ; the reads
  // of 32 lanes (one cycle for ds_read_b64) take units u, u+1 of 16
  // consecutive rows, 4 lines whose F values differ in bits 1-2.
  auto vt_at = [](int row, int unit) {
    const int L = row >> 2;
    const int F = ((L & 3) << 1) | (((L >> 2) & 3) << 3) | ((L >> 4) & 1);
    return 128 * L + 4 * ((8 * (row & 3) + unit) ^ F);
  };

  f32x4 acc[NRB][NDB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int i = 0; i < NDB; ++i) acc[rb][i] = f32x4{};
  float m_run[NRB], l_run[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    m_run[rb] = kMaxInit;
    l_run[rb] = 0.f;
  }

  // K: without STREAM, loaded straight into the A operand (kr[kb * KSTEPS + s]
  // holds 16 bytes of key 16*kb + c16 at dims 32*s + 8*q4: each load covers
  // 64 bytes of 16 rows).  With STREAM, rows are loaded whole (CR consecutive
  // lanes per row, full 128-byte lines, which non-temporal loads need) into
  // kr[i] = chunk u % CR of row u / CR, u = lane + 64*i, and staged through
  // the wave's K slab, chunk c of row r at c ^ kswz(r).
  u32x4 kr[KLD];
  u32x4 vr[VU][4];
  uint16_t* kl = k_lds + (STREAM ? w * 32 * D : 0);
  auto load_k = [&](int k0) {
    if constexpr (STREAM) {
#pragma unroll
      for (int i = 0; i < KLD; ++i) {
        const int u = lane + 64 * i, key = k0 + u / CR;
        u32x4 r = {0u, 0u, 0u, 0u};
        if (key < w1) r = ld16(Kb + (size_t)key * k_tok + 8 * (u % CR));
        kr[i] = r;
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int key = k0 + 16 * kb + c16;
        const bool ok = key < w1;
        const uint16_t* p = Kb + (size_t)(ok ? key : 0) * k_tok + 8 * q4;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
          u32x4 r = {0u, 0u, 0u, 0u};
          if (ok) r = *(const u32x4*)(p + 32 * s);
          kr[kb * KSTEPS + s] = r;
        }
      }
    }
  };
  auto store_k = [&]() {
#pragma unroll
    for (int i = 0; i < KLD; ++i) {
      const int u = lane + 64 * i, row = u / CR;
      *(u32x4*)(kl + row * D + 8 * ((u % CR) ^ kswz(row))) = kr[i];
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
        if (key < w1) r = ld16(Vb + (size_t)key * v_tok + 8 * dc);
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
        *(u32x2*)(vl + vt_at(8 * dc + e, kq)) = pk;
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
    if constexpr (STREAM) {
      store_k();
      wave_lds_sync();
      if (kn < w1) {
        load_v(kn);
        load_k(kn);
      }
    } else {
      if (kn < w1) load_v(kn);
    }
    // S^T for keys k0 + 16*kb + 4*q4 + r (register r), query row 16rb + c16;
    // the A operand of k-step st: dims 32*st + 8*q4 of key 16*kb + c16.
    f32x4 s[NRB][2];
    if constexpr (STREAM) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int row = 16 * kb + c16;
#pragma unroll
        for (int st = 0; st < KSTEPS; ++st) {
          const u32x4 kf = *(const u32x4*)(kl + row * D + 8 * ((4 * st + q4) ^ kswz(row)));
#pragma unroll
          for (int rb = 0; rb < NRB; ++rb)
            s[rb][kb] = E::mma16(E::as8(kf), qf[rb][st], st == 0 ? f32x4{} : s[rb][kb]);
        }
      }
    } else {
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          s[rb][kb] = f32x4{};
#pragma unroll
          for (int st = 0; st < KSTEPS; ++st)
            s[rb][kb] = E::mma16(E::as8(kr[kb * KSTEPS + st]), qf[rb][st], s[rb][kb]);
        }
    }
    if constexpr (!STREAM)
      if (kn < w1) load_k(kn);
    if (kn > w1) {
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (k0 + 16 * kb + 4 * q4 + r >= w1) s[rb][kb][r] = -INFINITY;
    }
    float corr[NRB];
    typename E::v8 pf[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[rb][kb][r]);
      mx = xor32_max(xor16_max(mx));
      const float m_new = fmaxf(m_run[rb], mx * a.cx);
      corr[rb] = fast_exp2(m_run[rb] - m_new);
      m_run[rb] = m_new;
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = fast_exp2(fmaf(s[rb][kb][r], a.cx, -m_new));
          rs += p;
          s[rb][kb][r] = p;
        }
      l_run[rb] = fmaf(l_run[rb], corr[rb], rs);
      // P^T as the B operand: slot j < 4 <-> key 4*q4 + j, slot j >= 4 <-> key 16 + 4*q4 + j - 4.
      u32x4 pk;
      pk[0] = E::pack2(s[rb][0][0], s[rb][0][1]);
      pk[1] = E::pack2(s[rb][0][2], s[rb][0][3]);
      pk[2] = E::pack2(s[rb][1][0], s[rb][1][1]);
      pk[3] = E::pack2(s[rb][1][2], s[rb][1][3]);
      pf[rb] = E::as8(pk);
    }
    wave_lds_sync();
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const u32x2 lo = *(const u32x2*)(vl + vt_at(16 * db + c16, q4));
      const u32x2 hi = *(const u32x2*)(vl + vt_at(16 * db + c16, q4 + 4));
      const u32x4 av = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        acc[rb][db] *= corr[rb];
        acc[rb][db] = E::mma16(E::as8(av), pf[rb], acc[rb][db]);
      }
    }
    wave_lds_sync();
  }

  // ---- combine the 4 waves of this work item, one row block at a time ----
  const bool final_out = c0 == 0 && L <= a.chunk;
  const size_t part = (size_t)bg * a.nch + chunk_id;
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
    combine_rows<DV>(a, (float*)vt_lds, acc[rb], m_run[rb], xor32_sum(xor16_sum(l_run[rb])), row0, rb, b, g,
                     part, final_out);
}

// ---------------------------------------------------------------------------
// fp32 GQA split-KV decode: the work items and wave split of
// gqa_decode_kernel with full fp32 products on v_mfma_f32_16x16x4f32
// (A lane l holds A[l%16][l/16], B lane l holds B[l/16][l%16], C as
// 16x16x32).  Q.K contracts dims d = 16j + 4*q4 + e in step (j, e) with k
// index q4, so each lane's K and Q^T operands are float4 loads of dims
// 16j + 4*q4 .. +3.  P.V's B operand for step e is the score register e
// itself (keys 4*q4 + e of a 16-key block), and its A operand V[key][dim] is
// loaded per lane (16 lanes read 16 consecutive dims of one key row).  Up to
// 32 rows (2 row blocks).
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma16x16x4f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int D, int DV, int NRB>
__global__ __launch_bounds__(256, 1) void gqa_decode_f32_kernel(DecodeArgs a) {
  constexpr int NJ = D / 16;    // float4 groups of Q.K per lane
  constexpr int NDB = DV / 16;  // 16-dim output blocks
  static_assert(D % 64 == 0 && DV % 64 == 0 && NRB <= 2, "fp32 decode shape");
  __shared__ __attribute__((aligned(16))) float red[4 * 16 * DV + 4 * 16 * 2];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c16 = lane & 15, q4 = lane >> 4;
  __shared__ int sched[4 + 2 * kSchedMaxBatch];
  int b, g, chunk_id, L;
  if (!decode_item(a, sched, b, g, chunk_id, L)) return;
  const int bg = b * a.G + g;
  const int c0 = chunk_id * a.chunk;
  const int per_wave = ((min(L - c0, a.chunk) + 127) >> 7) << 5;
  const int w0 = c0 + w * per_wave;
  const int w1 = min(w0 + per_wave, L);
  const float* Q = (const float*)a.q;
  const size_t k_tok = (size_t)a.G * D, v_tok = (size_t)a.G * DV;
  const float* Kb = (const float*)a.k + ((size_t)b * a.Lk * a.G + g) * D;
  const float* Vb = (const float*)a.v + ((size_t)b * a.Lk * a.G + g) * DV;
  const int row0 = blockIdx.y * 16 * NRB;  // this row group's first row

  f32x4 qf[NRB][NJ];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    const int row = row0 + 16 * rb + c16;
    const bool rv = row < a.rows;
    int t = 0, h = 0;
    if (rv) row_to_head(a, g, row, t, h);
    const float* qrow = Q + ((size_t)(b * a.Lq + t) * a.Hq + h) * D;
#pragma unroll
    for (int j = 0; j < NJ; ++j) qf[rb][j] = rv ? *(const f32x4*)(qrow + 16 * j + 4 * q4) : f32x4{};
  }
  f32x4 acc[NRB][NDB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int i = 0; i < NDB; ++i) acc[rb][i] = f32x4{};
  float m_run[NRB], l_run[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    m_run[rb] = kMaxInit;
    l_run[rb] = 0.f;
  }

  for (int k0 = w0; k0 < w1; k0 += 32) {
    // S^T for keys k0 + 16*kb + 4*q4 + r, query row 16rb + c16.
    f32x4 s[NRB][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int key = k0 + 16 * kb + c16;
      const bool ok = key < w1;
      const float* kp = Kb + (size_t)(ok ? key : 0) * k_tok + 4 * q4;
      f32x4 kf[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) kf[j] = ok ? *(const f32x4*)(kp + 16 * j) : f32x4{};
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        s[rb][kb] = f32x4{};
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) s[rb][kb] = mfma16x16x4f32(kf[j][e], qf[rb][j][e], s[rb][kb]);
      }
    }
    // V[key 16kb + 4*q4 + e][dim 16i + c16] for the A operands of P.V
    float vv[2][4][NDB];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = k0 + 16 * kb + 4 * q4 + e;
        const bool ok = key < w1;
        const float* vp = Vb + (size_t)(ok ? key : 0) * v_tok + c16;
#pragma unroll
        for (int i = 0; i < NDB; ++i) vv[kb][e][i] = ok ? vp[16 * i] : 0.f;
      }
    if (k0 + 32 > w1) {
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (k0 + 16 * kb + 4 * q4 + r >= w1) s[rb][kb][r] = -INFINITY;
    }
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[rb][kb][r]);
      mx = xor32_max(xor16_max(mx));
      const float m_new = fmaxf(m_run[rb], mx * a.cx);
      const float corr = fast_exp2(m_run[rb] - m_new);
      m_run[rb] = m_new;
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = fast_exp2(fmaf(s[rb][kb][r], a.cx, -m_new));
          rs += p;
          s[rb][kb][r] = p;
        }
      l_run[rb] = fmaf(l_run[rb], corr, rs);
#pragma unroll
      for (int i = 0; i < NDB; ++i) {
        acc[rb][i] *= corr;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[rb][i] = mfma16x16x4f32(vv[kb][e][i], s[rb][kb][e], acc[rb][i]);
      }
    }
  }

  const bool final_out = c0 == 0 && L <= a.chunk;
  const size_t part = (size_t)bg * a.nch + chunk_id;
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
    combine_rows<DV>(a, red, acc[rb], m_run[rb], xor32_sum(xor16_sum(l_run[rb])), row0, rb, b, g, part,
                     final_out);
}

// ---------------------------------------------------------------------------
// Latent (MLA) decode: K = V = one shared latent cache row of D dims per key,
// the first DV dims acting as values.  One workgroup = one (chunk, batch)
// item; the two LDS stages (2 x 64 keys x 2D bytes) leave room for one
// workgroup per CU.
//   * Each 64-key tile is contiguous in HBM (64 rows x 2D bytes) and is copied
//     HBM -> LDS with buffer->LDS loads, 1 KiB per wave instruction; the next
//     tile is in flight while the current one is computed.
//   * Wave w forms S^T = K Q^T for keys [16w, 16w+16) of every tile with
//     v_mfma_f32_16x16x32_bf16 (K rows from LDS, Q^T in registers) and writes
//     it to LDS (1 KiB); after a barrier every wave reads the whole 64 x 16
//     score tile, runs the online softmax over it (the same values in every
//     wave) and computes O^T += V^T P^T for its DV/4 output dims over all 64
//     keys with v_mfma_f32_16x16x16_bf16, whose B operands are the shared
//     score blocks as they stand (the C layout of S^T is the B layout of
//     P^T) and whose A operands (V^T) come from the same LDS tile through
//     ds_read_b64_tr_b16.  The latent row is read from HBM once and from LDS
//     twice.
//   * Each wave ends with the finished (max, sum, O) of its dims: nothing is
//     combined across waves (a combine of four key-split partials through LDS
//     took ~2.6 us of the C5 step).
// LDS rows keep their 16-byte columns XOR-swizzled per row (within aligned
// groups of 8 or 16 columns), so that 16 lanes reading one column of 16 rows
// (K fragments) and 32 lanes reading two columns of 8 rows (transposing V
// reads) touch distinct banks.
// ---------------------------------------------------------------------------
template <int D>
struct LatentTile {
  static constexpr int BK = 64;                    // keys per tile
  static constexpr int ROWB = 2 * D;               // bytes per latent row
  static constexpr int NC = D / 8;                 // 16-byte columns per row
  static constexpr int STAGE_B = BK * ROWB;        // bytes per stage
  static constexpr int NLD = STAGE_B / (4 * 1024);  // 1 KiB loads per wave per tile
  static constexpr int GRP = (NC % 16 == 0) ? 16 : 8;  // swizzle group (columns)
  static_assert(NC % 8 == 0 && STAGE_B % 4096 == 0, "latent tile shape");
  // Row r's column XOR.  Row r starts at 16-byte bank unit (r*NC) % 16, which
  // is 0 when NC % 16 == 0 and 8*(r&1) when NC % 16 == 8.  K fragments
  // (ds_read_b128) have lane l read column 4e + l/16 of row l%16, and gfx950's
  // LDS serves lanes 0-7 with 24-31 and 8-15 with 16-23 in one cycle, so rows
  // r < 8 of column 4e and rows r + 8 of column 4e + 1 must take different
  // bank groups: XOR 2(r&7) (whole lines) or r&6 (half lines) sends the first
  // to even groups and the second to odd ones.  The transposing V^T reads
  // (32 lanes: an aligned column pair of 8 consecutive rows) stay distinct.
  __device__ static int swz(int r) { return GRP == 16 ? ((r & 7) << 1) : (r & 6); }
};

template <typename E, int D, int DV, bool STREAM>
__global__ __launch_bounds__(kDecThreads, 1) void mla_decode_kernel(DecodeArgs a) {
  using T = LatentTile<D>;
  constexpr int BK = T::BK, ROWB = T::ROWB, NLD = T::NLD, GRP = T::GRP;
  constexpr int KSTEPS = D / 32;  // 32-dim k-steps of Q.K
  constexpr int SPG = GRP / 4;    // k-steps per swizzle group
  constexpr int NDT = DV / 16;    // 16-dim output tiles
  constexpr int NDW = NDT / 4;    // output tiles of one wave
  constexpr int DPG = GRP / 2;    // output tiles per swizzle group
  static_assert(DV % 64 == 0 && DV <= D, "value dims are a prefix of the latent row");
  static_assert(KSTEPS % SPG == 0 && NDT % DPG == 0, "swizzle groups");
  __shared__ __attribute__((aligned(1024))) unsigned char smem0[T::STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char smem1[T::STAGE_B];
  __shared__ f32x4 sx[4 * 64];  // the tile's S^T blocks, one per wave, in MFMA C layout

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, q4 = lane >> 4;
  __shared__ int sched[4 + 2 * kSchedMaxBatch];
  int b, g, chunk_id, L;
  if (!decode_item(a, sched, b, g, chunk_id, L)) return;  // nothing past the length is read
  const int c0 = chunk_id * a.chunk;
  const int c1 = min(c0 + a.chunk, L);
  const int n_tiles = (c1 - c0 + BK - 1) / BK;

  // Q^T as the B operand: lane holds query row row0 + c16 (16 rows per row
  // group, blockIdx.y), dims 32*s + 8*q4 + [0,8).
  const int row = blockIdx.y * 16 + c16;
  typename E::v8 qf[KSTEPS];
  {
    const bool rv = row < a.rows;
    int t = 0, h = 0;
    if (rv) row_to_head(a, 0, row, t, h);
    const uint16_t* qrow = a.q + ((size_t)(b * a.Lq + t) * a.Hq + h) * D;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      u32x4 r = {0u, 0u, 0u, 0u};
      if (rv) r = *(const u32x4*)(qrow + 32 * s + 8 * q4);
      qf[s] = E::as8(r);
    }
  }
  const unsigned char* Kb = (const unsigned char*)a.k + (size_t)b * a.Lk * ROWB;

  // Buffer->LDS sources: load j of wave w fills 16-byte LDS unit
  // p = (NLD*w + j)*64 + lane = row*NC + slot with global column slot ^ swz(row).
  uint32_t voff[NLD];
#pragma unroll
  for (int j = 0; j < NLD; ++j) {
    const int p = (NLD * w + j) * 64 + lane, r = p / T::NC, slot = p % T::NC;
    voff[j] = r * ROWB + 16 * (slot ^ T::swz(r));
  }
  // K fragment of k-step s: row 16w + c16, column 4s + q4, i.e. group s / SPG,
  // column 4*(s % SPG) + q4 within it.
  uint32_t offK[SPG];
  {
    const int r = 16 * w + c16;
#pragma unroll
    for (int e = 0; e < SPG; ++e) offK[e] = r * ROWB + 16 * ((4 * e + q4) ^ T::swz(r));
  }
  // Transposing V^T read for output tile dt (dims 16*dt + [0,16)) and key
  // block kb (keys 16kb + 4*q4 + [0,4)): lane s of each 16-lane group points
  // at row 16kb + 4*q4 + s/4, dims 16*dt + 4*(s%4) + [0,4).  The swizzle of a
  // row depends on it modulo 16 only, so key block kb is offV + 16*kb rows.
  uint32_t offV[DPG];
  {
    const int r = 4 * q4 + (c16 >> 2);
#pragma unroll
    for (int e = 0; e < DPG; ++e)
      offV[e] = r * ROWB + 16 * ((2 * e + ((c16 & 3) >> 1)) ^ T::swz(r)) + 8 * (c16 & 1);
  }

  // acc[i] = O^T[dims 16*(NDW*w + i) + 4*q4 + r][row c16]
  f32x4 acc[NDW];
#pragma unroll
  for (int i = 0; i < NDW; ++i) acc[i] = f32x4{};
  float m_run = kMaxInit, l_run = 0.f;

  auto issue = [&](int t, unsigned char* ks) {
    const int k0 = c0 + t * BK;
    // Rows at or past c1 read as 0; a tile past the chunk reads nothing.
    // (readfirstlane: the clamp is computed on the vector unit, and a vector
    // operand of the buffer descriptor would need a waterfall loop.)
    const uint32_t bytes = __builtin_amdgcn_readfirstlane(max(0, min(BK, c1 - k0)) * ROWB);
    const rsrc_t rs = make_rsrc(Kb + (size_t)k0 * ROWB, bytes);
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      // STREAM: non-temporal loads for caches past the MALL (as in gqa_decode_kernel)
      if constexpr (STREAM) buffer_load_lds16_nt(rs, ks + (NLD * w + j) * 1024, voff[j]);
      else buffer_load_lds16(rs, ks + (NLD * w + j) * 1024, voff[j]);
    }
  };

  // One tile: wave w forms S^T for its 16 keys and shares it; every wave runs
  // the softmax over all 64 keys (the same values in every wave) and
  // multiplies its own NDW output tiles over all 64 keys.
  auto compute = [&](int t, const unsigned char* ks) {
    const int k0 = c0 + t * BK;
    // s[r] = S^T[key k0 + 16w + 4*q4 + r][row c16]
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < KSTEPS; ++st) {
      const typename E::v8 kf = E::as8(*(const u32x4*)(ks + offK[st % SPG] + 16 * GRP * (st / SPG)));
      s = E::mma16(kf, qf[st], s);
    }
    // Keys at or past c1 -> -inf, selected on every tile (a no-op on full
    // ones) so that the score passes through the vector ALU before its LDS
    // store.  Stored straight from the MFMA accumulator, one instruction
    // after the last MFMA, the value written was sometimes not the finished
    // one when other waves shared the SIMD's matrix pipe (ranks <= 256 run
    // 2-7 workgroups per CU): wrong scores for 4 keys of a row, changing from
    // run to run; 32 wait states before the store, or one workgroup per CU,
    // made every result exact.  A vector-ALU read of an MFMA result is
    // covered by the compiler's MFMA hazard waits; the LDS store's data read
    // was not.
    {
      const int lim = c1 - (k0 + 16 * w + 4 * q4);
#pragma unroll
      for (int r = 0; r < 4; ++r) s[r] = r < lim ? s[r] : -INFINITY;
    }
    sx[w * 64 + lane] = s;
    stage_barrier();
    f32x4 sk[4];  // sk[kb][r] = S^T[key k0 + 16kb + 4*q4 + r][row c16]
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) sk[kb] = sx[kb * 64 + lane];
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) mx = fmaxf(mx, fmaxf(fmaxf(sk[kb][0], sk[kb][1]), fmaxf(sk[kb][2], sk[kb][3])));
    mx = xor16_max(mx);
    const float mc = xor32_max(mx) * a.cx;
    if (wave_any(mc > m_run + kRescaleLog2)) {
      const float m_new = fmaxf(m_run, mc);
      const float corr = fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= corr;
#pragma unroll
      for (int i = 0; i < NDW; ++i) acc[i] *= corr;
    }
    s16x4 pb[4];
    float ls = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = fast_exp2(fmaf(sk[kb][r], a.cx, -m_run));
      ls += (p[0] + p[1]) + (p[2] + p[3]);
      const u32x2 pk = {E::pack2(p[0], p[1]), E::pack2(p[2], p[3])};
      pb[kb] = __builtin_bit_cast(s16x4, pk);
    }
    l_run += ls;
#pragma unroll
    for (int i = 0; i < NDW; ++i) {
      const int dt = NDW * w + i;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const u32x2 av = lds_read_tr16(ks + 16 * kb * ROWB + offV[dt % DPG] + 16 * GRP * (dt / DPG));
        acc[i] = E::mma16k16(__builtin_bit_cast(s16x4, av), pb[kb], acc[i]);
      }
    }
  };

  // Tile t lives in stage t % 2.  Before computing tile t: this wave's loads
  // of it have landed (vmcnt counts loads in issue order and only tile t+1's
  // may still be pending), then the barrier makes every wave's loads visible
  // (each wave reads V^T rows of all four waves).  After computing it, a
  // barrier lets tile t+2 be loaded into the same stage.
  // Every path issues the same sequence of loads (tiles past the chunk are
  // empty) and the loop has no early exit, so the compiler can tell that at
  // each read of a stage the NLD most recent loads target the other stage,
  // and adds no wait of its own.
  // Prologue: Q's loads are waited for while tile 0 is in flight, so that no
  // load into registers is pending at the loop (the compiler would otherwise
  // wait for every outstanding load, tile 1's included, before entering it).
  __builtin_amdgcn_sched_barrier(0);
  issue(0, smem0);
  wait_vmcnt<NLD>();
  issue(1, smem1);
  for (int t = 0; t < n_tiles; t += 2) {
    wait_vmcnt<NLD>();
    stage_barrier();
    compute(t, smem0);
    stage_barrier();
    issue(t + 2, smem0);
    wait_vmcnt<NLD>();
    stage_barrier();
    if (t + 1 < n_tiles) compute(t + 1, smem1);
    stage_barrier();
    issue(t + 3, smem1);
  }
  wait_vmcnt<0>();  // the trailing (empty) tile loads still write LDS

  // Every wave holds the same (max, sum) and the whole output of its dims:
  // no combine across waves.
  l_run = xor16_sum(l_run);
  l_run = xor32_sum(l_run);
  if (row < a.rows) {
    const size_t part = (size_t)b * a.nch + chunk_id;
    const bool final_out = c0 == 0 && L <= a.chunk;
#pragma unroll
    for (int i = 0; i < NDW; ++i)
      emit_row_quad(a, b, 0, row, 16 * (NDW * w + i) + 4 * q4, part, final_out, m_run, l_run, acc[i]);
  }
}

// Exact merge of the chunk partials of one (batch, group, query row):
// M = max_c m_c, O = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c
// (attention_splitkv.py:236-245, with unnormalised partials).  One thread per
// 4 output dims.  The partials are taken in batches of kMergeBatch chunks whose
// loads (m, l and 4 dims of O per chunk) are all issued before any is used, so
// a batch costs one memory round trip (the first one overlapping the length
// load); batches are combined online (running max, rescaled sums).  Sequences that fit one chunk were finished by the
// chunk kernel; empty sequences (length 0, no chunk ran) get a zero output and
// LSE = +inf (attention_xla.py:417-420).
constexpr int kMergeThreads = 128;
constexpr int kMergeBatch = 16;
__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(DecodeArgs a) {
  const int nq = a.dv / 4;
  const long gid = (long)blockIdx.x * kMergeThreads + threadIdx.x;
  const long item = gid / nq;
  const int u = (int)(gid % nq);
  if (item >= (long)a.B * a.G * a.rows) return;
  const int bg = (int)(item / a.rows), r = (int)(item % a.rows);
  const int b = bg / a.G, g = bg % a.G;
  const size_t base = (size_t)bg * a.nch;
  const float* ml = a.ws_ml + (base * a.rows + r) * 2;  // chunk c at ml[c * ml_stride]
  const size_t ml_stride = (size_t)a.rows * 2;
  const float* po = a.ws_o + (base * a.rows + r) * a.dv + 4 * u;  // chunk c at po[c * o_stride]
  const size_t o_stride = (size_t)a.rows * a.dv;
  // The sequence length is needed only after the first batch's loads are
  // issued: partial addresses are clamped to the workspace's a.nch chunks,
  // and slots at or past this sequence's chunk count n (never written by this
  // call) are dropped by selects, so whatever they hold cannot leak in.
  // (A buffer load of the length: unconditional, so nothing waits for it
  // before the partial loads; without lengths the buffer is empty.)
  const int len_raw = (int)__builtin_amdgcn_raw_buffer_load_b32(
      make_rsrc(a.lengths, a.lengths ? (uint32_t)a.B * 4u : 0u), b * 4, 0, 0);
  float M = kMaxInit, den = 0.f;
  f32x4 num = {0.f, 0.f, 0.f, 0.f};
  float mv[kMergeBatch], lv[kMergeBatch];
  f32x4 ov[kMergeBatch];
  auto load_batch = [&](int c0) {
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      const size_t c = (size_t)min(c0 + i, a.nch - 1);
      mv[i] = ml[c * ml_stride];
      lv[i] = ml[c * ml_stride + 1];
      ov[i] = *(const f32x4*)(po + c * o_stride);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the batch ahead of the arithmetic
  };
  auto add_batch = [&](int c0, int n) {
    float bm = M;
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i)
      if (c0 + i < n) bm = fmaxf(bm, mv[i]);
    const float sc = fast_exp2(M - bm);
    M = bm;
    den *= sc;
    num *= sc;
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      if (c0 + i < n) {
        const float wt = fast_exp2(mv[i] - M);
        den = fmaf(wt, lv[i], den);
        num += wt * ov[i];
      }
    }
  };
  load_batch(0);
  const int L = a.lengths ? min(a.Lk, max(len_raw, 0)) : a.Lk;  // as seq_len
  const int n = (L + a.chunk - 1) / a.chunk;
  if (n == 1) return;  // the chunk kernel wrote this row's output
  add_batch(0, n);
  for (int c0 = kMergeBatch; c0 < n; c0 += kMergeBatch) {
    load_batch(c0);
    add_batch(c0, n);
  }
  int t, h;
  row_to_head(a, g, r, t, h);
  const float inv = den > 0.f ? 1.f / den : 0.f;
  const size_t oi = ((size_t)(b * a.Lq + t) * a.Hq + h) * a.dv + 4 * u;
  if (a.o32) {
    *(f32x4*)(a.o32 + oi) = num * inv;
  } else {
    const u32x2 pk = a.f16 ? u32x2{F16Fmt::pack2(num[0] * inv, num[1] * inv), F16Fmt::pack2(num[2] * inv, num[3] * inv)}
                           : u32x2{Bf16Fmt::pack2(num[0] * inv, num[1] * inv), Bf16Fmt::pack2(num[2] * inv, num[3] * inv)};
    *(u32x2*)(a.o + oi) = pk;
  }
  if (a.lse && u == 0)
    a.lse[((size_t)b * a.Hq + h) * a.Lq + t] = den > 0.f ? (M + __log2f(den)) * kLn2 : INFINITY;
}

// Keys per work item when the caller passes chunk = 0: the smallest power of
// two in [128, 2048] that leaves at most `items` (chunk, batch, group) work
// items at full capacity.  Longer items amortise the per-item start-up (Q
// fragments, the cross-wave combine, partial writes); the item target keeps
// short batches spread over every CU.  Measured on MI355X (GQA, 32 query
// heads over 8 KV heads, D = 128, ragged lengths): ~1024 items at capacity is
// best or within 1% of best for 32 x 8192, 64 x 4096 and full-length 32 x
// 8192 (2048-key chunks) and for 4 x 32768 (1024-key chunks; 2048-key chunks
// leave too few items and take 1.75x as long); the latent decode is fastest
// with ~256 (256-key chunks for 16 x 4096).
constexpr int64_t kGqaItems = 1024;
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

template <auto K>
static int run_decode(DecodeArgs& a, void* workspace, size_t ws_bytes,
                      hipStream_t stream, const char* name) {
  const size_t need = ws_size(a.B, a.G, a.rows, a.Lk, a.dv, a.chunk);
  if (!workspace || ws_bytes < need) return fail(PJX_ERR_WORKSPACE, "decode: workspace missing or too small");
  const size_t parts = (size_t)a.B * a.G * a.nch * a.rows;
  a.ws_o = (float*)workspace;
  a.ws_ml = a.ws_o + parts * a.dv;
  const long blocks = (long)a.B * a.G * a.nch;
  const long groups = ((long)a.rows + a.rpg - 1) / a.rpg;
  if (blocks > 0x7fffffffL || groups > 65535 || (long)a.B * a.G * a.rows > 0x7fffffffL)
    return fail(PJX_ERR_INVALID, "decode: grid too large");
  launch_kernel<K>(dim3((unsigned)blocks, (unsigned)groups), dim3(kDecThreads), 0, stream, a);
  int rc = check_launch(name);
  if (rc) return rc;
  const long merge_threads = (long)a.B * a.G * a.rows * (a.dv / 4);
  launch_kernel<decode_merge_kernel>(dim3((unsigned)((merge_threads + kMergeThreads - 1) / kMergeThreads)),
                     dim3(kMergeThreads), 0, stream, a);
  return check_launch(name);
}

// 16-row MFMA column blocks per row group of a GQA decode launch: up to 4 (64
// rows, the reference's largest packed tile, attention_splitkv.py:155-170) at
// head dims <= 128 in bf16 / fp16, else 2; more rows run as several row groups.
static int gqa_row_blocks(int64_t rows, int64_t head_dim, int64_t v_dim, bool f32) {
  const int64_t max_nrb = (f32 || head_dim > 128 || v_dim > 128) ? 2 : 4;
  const int64_t need = std::min<int64_t>((rows + kRows - 1) / kRows, max_nrb);
  return need <= 1 ? 1 : need <= 2 ? 2 : 4;
}

// One (D, DV) pair of the 16-bit GQA decode with nrb 16-row blocks per row group.
template <typename E, int D, int DV, bool STREAM>
static int run_gqa_nrb(DecodeArgs& a, int nrb, void* ws, size_t ws_bytes, hipStream_t s, const char* who) {
  if (nrb == 1) return run_decode<gqa_decode_kernel<E, D, DV, 1, STREAM>>(a, ws, ws_bytes, s, who);
  if (nrb == 2) return run_decode<gqa_decode_kernel<E, D, DV, 2, STREAM>>(a, ws, ws_bytes, s, who);
  if constexpr (D <= 128 && DV <= 128) return run_decode<gqa_decode_kernel<E, D, DV, 4, STREAM>>(a, ws, ws_bytes, s, who);
  return fail(PJX_ERR_INVALID, "decode: row blocks");
}

template <typename E, int D, int DV>
static int run_gqa_dims(DecodeArgs& a, int nrb, bool streamed, void* ws, size_t ws_bytes, hipStream_t s,
                        const char* who) {
  return streamed ? run_gqa_nrb<E, D, DV, true>(a, nrb, ws, ws_bytes, s, who)
                  : run_gqa_nrb<E, D, DV, false>(a, nrb, ws, ws_bytes, s, who);
}

template <int D, int DV>
static int run_gqa_f32_dims(DecodeArgs& a, int nrb, void* ws, size_t ws_bytes, hipStream_t s, const char* who) {
  return nrb == 1 ? run_decode<gqa_decode_f32_kernel<D, DV, 1>>(a, ws, ws_bytes, s, who)
                  : run_decode<gqa_decode_f32_kernel<D, DV, 2>>(a, ws, ws_bytes, s, who);
}

// The GQA decode at (head_dim, v_dim), each in {64, 128, 256}: format E (bf16 /
// fp16), or fp32 when F32.
template <typename E, bool F32>
static int run_gqa(DecodeArgs& a, int head_dim, int v_dim, int nrb, bool streamed, void* ws, size_t ws_bytes,
                   hipStream_t s, const char* who) {
#define PJX_GQA_DIMS(D, DV)                                                                   \
  if (head_dim == D && v_dim == DV) {                                                         \
    if constexpr (F32) return run_gqa_f32_dims<D, DV>(a, nrb, ws, ws_bytes, s, who);            \
    else return run_gqa_dims<E, D, DV>(a, nrb, streamed, ws, ws_bytes, s, who);               \
  }
  PJX_GQA_DIMS(64, 64) PJX_GQA_DIMS(64, 128) PJX_GQA_DIMS(64, 256)
  PJX_GQA_DIMS(128, 64) PJX_GQA_DIMS(128, 128) PJX_GQA_DIMS(128, 256)
  PJX_GQA_DIMS(256, 64) PJX_GQA_DIMS(256, 128) PJX_GQA_DIMS(256, 256)
#undef PJX_GQA_DIMS
  return fail(PJX_ERR_INVALID, "decode: head_dim and v_dim must be 64, 128 or 256");
}

// The latent decode (format E) at one (rank, v_dim); STREAM instances when
// `streamed`.
template <typename E, bool STREAM>
static int run_mla_rank(DecodeArgs& a, int64_t rank, int64_t v_dim, void* ws, size_t ws_bytes, hipStream_t s) {
  const char* who = "pjx_mla_decode";
  if (rank == 576 && v_dim == 512) return run_decode<mla_decode_kernel<E, 576, 512, STREAM>>(a, ws, ws_bytes, s, who);
  if (rank == 576 && v_dim == 576) return run_decode<mla_decode_kernel<E, 576, 576, STREAM>>(a, ws, ws_bytes, s, who);
  if (rank == 512 && v_dim == 512) return run_decode<mla_decode_kernel<E, 512, 512, STREAM>>(a, ws, ws_bytes, s, who);
  if (rank == 256 && v_dim == 256) return run_decode<mla_decode_kernel<E, 256, 256, STREAM>>(a, ws, ws_bytes, s, who);
  if (rank == 128 && v_dim == 128) return run_decode<mla_decode_kernel<E, 128, 128, STREAM>>(a, ws, ws_bytes, s, who);
  if (rank == 64 && v_dim == 64) return run_decode<mla_decode_kernel<E, 64, 64, STREAM>>(a, ws, ws_bytes, s, who);
  return fail(PJX_ERR_INVALID,
              "pjx_mla_decode: supported (rank, v_dim): (576,512), (576,576), (512,512), (256,256), (128,128), (64,64)");
}

template <typename E>
static int run_mla_h16(DecodeArgs& a, int64_t rank, int64_t v_dim, bool streamed, void* ws, size_t ws_bytes,
                       hipStream_t s) {
  return streamed ? run_mla_rank<E, true>(a, rank, v_dim, ws, ws_bytes, s)
                  : run_mla_rank<E, false>(a, rank, v_dim, ws, ws_bytes, s);
}

// Whether the 16-bit GQA and latent decodes stream the cache with
// non-temporal loads (the STREAM kernels).  Ordinary loads leave the cache in the 256 MB MALL, which
// repeated calls over a cache that (nearly) fits then hit: measured +3% to
// +17% for STREAM at 537 MB of capacity (~290 MB valid); past that, STREAM
// reads faster (-4% to -9% at 1 GB and more).  The lengths stay on the device,
// so the rule uses the capacity: STREAM above kStreamBytes (3x the MALL).
// The latent decode reads every cached row whole (no ragged tail in the
// measured cases) and crosses over earlier: STREAM measured +1% at 302 MB and
// -10% at 604 MB of latent (R = 576), so its threshold is kStreamBytesLatent.
// PJX_DECODE_STREAM=0 / =1 in the environment forces either kernel.
constexpr int64_t kStreamBytes = (int64_t)768 << 20;
constexpr int64_t kStreamBytesLatent = (int64_t)512 << 20;
static bool decode_streams_kv(int64_t cache_bytes, int64_t threshold) {
  const char* env = getenv("PJX_DECODE_STREAM");
  if (env && env[0] == '0' && env[1] == '\0') return false;
  if (env && env[0] == '1' && env[1] == '\0') return true;
  return cache_bytes > threshold;
}

// Argument checks shared by pjx_splitkv_decode and pjx_splitkv_decode_static
// (everything but the pointers and the workspace); resolves chunk = 0.
static int check_gqa_decode(const char* who, int dtype, int64_t batch, int64_t q_len, int64_t kv_len,
                            int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t v_dim,
                            float sm_scale, int64_t* chunk) {
  char buf[256];
  auto bad = [&](const char* what) {
    snprintf(buf, sizeof(buf), "%s: %s", who, what);
    return fail(PJX_ERR_INVALID, buf);
  };
  if (dtype != PJX_DTYPE_BF16 && dtype != PJX_DTYPE_F16 && dtype != PJX_DTYPE_F32)
    return bad("dtype must be PJX_DTYPE_BF16, PJX_DTYPE_F16 or PJX_DTYPE_F32");
  if (batch < 0 || q_len <= 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads)
    return bad("bad sizes");
  auto width = [](int64_t d) { return d == 64 || d == 128 || d == 256; };
  if (!width(head_dim) || !width(v_dim)) return bad("head_dim and v_dim must be 64, 128 or 256");
  if (!(sm_scale > 0.f)) return bad("sm_scale must be > 0");
  if (*chunk == 0) *chunk = auto_chunk(batch, kv_heads, kv_len, kGqaItems);
  if (*chunk < 128 || *chunk % 128) return bad("chunk must be a positive multiple of 128");
  const int64_t rows = (q_heads / kv_heads) * q_len;
  if (kv_len > (1 << 30) || batch * kv_len * kv_heads * std::max(head_dim, v_dim) > ((int64_t)1 << 40) ||
      rows > (1 << 20) || batch * q_heads * q_len * std::max(head_dim, v_dim) > ((int64_t)1 << 40))
    return bad("sizes out of range");
  return PJX_OK;
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
                                  int64_t kv_heads, int64_t head_dim, int64_t v_dim, float sm_scale,
                                  int64_t chunk, void* stream) {
  clear_error();
  const char* who = "pjx_splitkv_decode";
  const int vrc = check_gqa_decode(who, dtype, batch, q_len, kv_len, q_heads, kv_heads, head_dim, v_dim, sm_scale,
                                   &chunk);
  if (vrc != PJX_OK) return vrc;
  // an empty cache (kv_len == 0) may come as null pointers
  if (!q || !o || (batch * kv_len > 0 && (!k || !v))) return fail(PJX_ERR_INVALID, "pjx_splitkv_decode: null pointer");
  const bool f32 = dtype == PJX_DTYPE_F32;
  if (batch == 0) return PJX_OK;
  if (kv_len == 0)
    return write_keyless(o, lse, (size_t)(batch * q_len * q_heads * v_dim), f32, (size_t)(batch * q_heads * q_len),
                         (hipStream_t)stream, who);
  const int64_t rows = (q_heads / kv_heads) * q_len;
  DecodeArgs a = {};
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
  a.lengths = kv_lengths; a.lse = lse;
  if (f32)
    a.o32 = (float*)o;
  else
    a.o = (uint16_t*)o;
  a.f16 = dtype == PJX_DTYPE_F16;
  a.B = (int)batch; a.Lq = (int)q_len; a.Lk = (int)kv_len; a.Hq = (int)q_heads; a.G = (int)kv_heads;
  a.rows = (int)rows; a.fold = 0; a.chunk = (int)chunk;
  a.nch = (int)std::max<int64_t>((kv_len + chunk - 1) / chunk, 1);
  a.dv = (int)v_dim; a.cx = sm_scale * kLog2e;
  const int nrb = gqa_row_blocks(rows, head_dim, v_dim, f32);
  a.rpg = kRows * nrb;
  hipStream_t s = (hipStream_t)stream;
  const int d = (int)head_dim, dv = (int)v_dim;
  const bool streamed = !f32 && decode_streams_kv(batch * kv_len * kv_heads * (head_dim + v_dim) * 2, kStreamBytes);
  if (f32) return run_gqa<Bf16Fmt, true>(a, d, dv, nrb, false, workspace, workspace_bytes, s, who);
  return a.f16 ? run_gqa<F16Fmt, false>(a, d, dv, nrb, streamed, workspace, workspace_bytes, s, who)
               : run_gqa<Bf16Fmt, false>(a, d, dv, nrb, streamed, workspace, workspace_bytes, s, who);
}

// ---------------------------------------------------------------------------
// Split-KV decode without allocation: the partials live in `scratch`, a
// library-held device array (one copy per GPU, kept until the process ends),
// for callers that cannot allocate (graph capture, serving loops).  Every call
// on a GPU shares that GPU's array: calls that overlap on one GPU race.  No
// part of it needs clearing: the chunk kernel writes every partial the merge
// reads in the same call.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = (size_t)PJX_DECODE_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of the current device's `scratch` (the name itself is only a
// host-side stand-in), looked up on the first call on each device.
static int scratch_ptr(void** out, const char* who) {
  char buf[256];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    snprintf(buf, sizeof(buf), "%s: no usable current device (%s)", who, hipGetErrorString(e));
    return fail(PJX_ERR_LAUNCH, buf);
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      snprintf(buf, sizeof(buf), "%s: hipGetSymbolAddress(scratch) failed: %s", who, hipGetErrorString(e));
      return fail(PJX_ERR_LAUNCH, buf);
    }
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return PJX_OK;
}

extern "C" int pjx_splitkv_decode_static(int dtype, const void* q, const void* k, const void* v,
                                         const int32_t* kv_lengths, void* o, float* lse,
                                         int64_t batch, int64_t q_len, int64_t kv_len,
                                         int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                         int64_t v_dim, float sm_scale, int64_t chunk, void* stream) {
  clear_error();
  const char* who = "pjx_splitkv_decode_static";
  // every argument check of pjx_splitkv_decode first, then the size of the partials
  const int vrc = check_gqa_decode(who, dtype, batch, q_len, kv_len, q_heads, kv_heads, head_dim, v_dim, sm_scale,
                                   &chunk);
  if (vrc != PJX_OK) return vrc;
  if (batch == 0) return PJX_OK;
  const size_t need = ws_size(batch, kv_heads, (q_heads / kv_heads) * q_len, kv_len, v_dim, chunk);
  if (need > kScratchBytes) {
    char buf[256];
    snprintf(buf, sizeof(buf), "%s: these sizes need %zu bytes of partials, more than the %zu-byte "
             "scratch the library holds; call pjx_splitkv_decode with a workspace", who, need, kScratchBytes);
    return fail(PJX_ERR_WORKSPACE, buf);
  }
  void* ws = nullptr;
  const int rc = scratch_ptr(&ws, who);
  if (rc != PJX_OK) return rc;
  return pjx_splitkv_decode(dtype, q, k, v, kv_lengths, o, lse, ws, kScratchBytes, batch, q_len, kv_len,
                            q_heads, kv_heads, head_dim, v_dim, sm_scale, chunk, stream);
}

extern "C" int pjx_mla_decode(int dtype, const void* q, const void* cache,
                              const int32_t* kv_lengths, void* o, float* lse, void* workspace,
                              size_t workspace_bytes, int64_t batch, int64_t q_len,
                              int64_t heads, int64_t kv_len, int64_t rank, int64_t v_dim,
                              float sm_scale, int64_t chunk, void* stream) {
  clear_error();
  if (dtype != PJX_DTYPE_BF16 && dtype != PJX_DTYPE_F16)
    return fail(PJX_ERR_INVALID, "pjx_mla_decode: dtype must be PJX_DTYPE_BF16 or PJX_DTYPE_F16");
  // an empty cache (kv_len == 0) may come as a null pointer
  if (!q || !o || (batch * kv_len > 0 && !cache)) return fail(PJX_ERR_INVALID, "pjx_mla_decode: null pointer");
  if (batch < 0 || q_len <= 0 || heads <= 0 || kv_len < 0) return fail(PJX_ERR_INVALID, "pjx_mla_decode: bad sizes");
  if (q_len * heads > (1 << 20)) return fail(PJX_ERR_INVALID, "pjx_mla_decode: Lq*H must be <= 2^20");
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
  a.rpg = kRows;  // one 16-row MFMA column block per row group
  hipStream_t s = (hipStream_t)stream;
  if (batch == 0) return PJX_OK;
  if (kv_len == 0)
    return write_keyless(o, lse, (size_t)(batch * q_len * heads * v_dim), false, (size_t)(batch * heads * q_len), s,
                         "pjx_mla_decode");
  a.f16 = dtype == PJX_DTYPE_F16;
  // the latent is K and V at once: capacity B * S * R 16-bit values
  const bool streamed = decode_streams_kv(batch * kv_len * rank * 2, kStreamBytesLatent);
  return a.f16 ? run_mla_h16<F16Fmt>(a, rank, v_dim, streamed, workspace, workspace_bytes, s)
               : run_mla_h16<Bf16Fmt>(a, rank, v_dim, streamed, workspace, workspace_bytes, s);
}
