// Definitions shared by the flash-attention forward kernels of
// flash_fwd.hip and flash_bias_ring.hip: the argument block, the per-block
// geometry, the bias loader and the bf16 K/V tile layout.
#pragma once

#include "attn_mods.h"
#include "pjx_common.h"
#include "pjx_internal.h"

namespace pjx {

struct FlashArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  const int32_t* kv_lengths;
  const float* bias;
  long bias_bstride;  // elements between batch slices of the bias (0: broadcast)
  long bias_hstride;  // elements between head slices of the bias (0: broadcast)
  int B, Lq, Lk, Hq, Hkv;
  int q_valid, kv_valid, causal;
  float scale;
  int n_qtiles;
  int dv;       // output row width (elements per head); the wide kernels' V width
  int ext;      // 0: none; 1: interval masks in `m`; 2: also segment ids / score modifiers
  int f16;      // 16-bit inputs are fp16 (else bf16); read by the host-side launchers only
  ScoreMods m;
};

constexpr int kBQ = 128;
constexpr int kThreads = 256;

// fp32 forward at head dim 256 (flash_f32_wide.hip).  Returns a PJX_* status.
int launch_flash_f32_wide(const FlashArgs& a, hipStream_t s);

// Per-block geometry shared by both dtype paths.
struct BlockGeom {
  int b, h, hkv, q0, qw, qi;
  int q_hi;     // rows >= q_hi are fully masked (QKVLengthMask / Lq)
  int kv_end;   // keys >= kv_end are masked (KVLenMask, QKVLengthMask, Lk)
  int kv_stop;  // keys the block visits (kv_end, clipped causally)
  int kv_begin; // first key the block visits (a multiple of the key tile)
};

// idx: the block's index in the (q tile, batch, head) grid (blockIdx.x unless
// the grid carries a further factor).
__device__ __forceinline__ BlockGeom block_geom(const FlashArgs& a, int idx) {
  BlockGeom g;
  const int BH = a.B * a.Hq;
  const int bh = idx % BH;
  const int qt = a.n_qtiles - 1 - idx / BH;
  g.b = bh / a.Hq;
  g.h = bh % a.Hq;
  g.hkv = g.h / (a.Hq / a.Hkv);
  g.q0 = qt * kBQ;
  const int w = threadIdx.x >> 6;
  g.qw = g.q0 + 32 * w;
  g.qi = g.qw + (threadIdx.x & 31);
  g.q_hi = min(a.Lq, a.q_valid);
  int kv_end = min(a.Lk, a.kv_valid);
  if (a.kv_lengths) kv_end = min(kv_end, max(a.kv_lengths[g.b], 0));
  g.kv_end = kv_end;
  int stop = kv_end;
  if (g.q0 >= g.q_hi) {
    stop = 0;
  } else if (a.causal) {
    stop = min(stop, min(g.q0 + kBQ, g.q_hi));
  }
  g.kv_stop = stop;
  g.kv_begin = 0;
  return g;
}

__device__ __forceinline__ BlockGeom block_geom(const FlashArgs& a) { return block_geom(a, blockIdx.x); }

// With extended masks: the block's key range [kv_begin, kv_stop) from the
// interval bounds of its first and last row (both bounds are monotone in the
// row), kv_begin rounded down to the key tile.
__device__ __forceinline__ void ext_block_range(const FlashArgs& a, BlockGeom& g, int tile) {
  g.kv_begin = 0;
  if (g.q0 >= g.q_hi) {
    g.kv_stop = 0;
    return;
  }
  int lo0, hi0, lo1, hi1;
  const int q_last = min(g.q0 + kBQ, g.q_hi) - 1;
  row_bounds(a.m, a.causal, g.b, g.kv_end, g.q_hi, g.q0, lo0, hi0);
  row_bounds(a.m, a.causal, g.b, g.kv_end, g.q_hi, q_last, lo1, hi1);
  g.kv_begin = (max(lo0, 0) / tile) * tile;
  g.kv_stop = max(min(hi1 + 1, g.kv_end), 0);
}

// Per-wave view of the extended masks for a wave owning rows qw .. qw+31 and
// a lane owning row qi (S^T layout: one query per lane).
struct ExtRows {
  int lo, hi;          // this lane's key interval
  int lo_first, hi_first;  // interval of the wave's first row
  int lo_last, hi_last;    // interval of the wave's last existing row
  bool any;            // the wave has a row < q_hi
  int segq;            // this row's segment id
  HeadMods hm;
};

__device__ __forceinline__ ExtRows ext_rows(const FlashArgs& a, const BlockGeom& g) {
  ExtRows e;
  row_bounds(a.m, a.causal, g.b, g.kv_end, g.q_hi, g.qi, e.lo, e.hi);
  e.any = g.qw < g.q_hi;
  const int ql = min(g.qw + 31, g.q_hi - 1);
  row_bounds(a.m, a.causal, g.b, g.kv_end, g.q_hi, g.qw, e.lo_first, e.hi_first);
  row_bounds(a.m, a.causal, g.b, g.kv_end, g.q_hi, ql, e.lo_last, e.hi_last);
  e.segq = (a.m.seg_q && g.qi < a.Lq) ? a.m.seg_q[(size_t)g.b * a.Lq + g.qi] : 0;
  e.hm = head_mods(a.m, g.h);
  return e;
}

// Segment ids of 4 consecutive positions kk .. kk+3 (kk a multiple of 4) of
// batch b in ids [B, L] (0 past L).
__device__ __forceinline__ int4 seg4(const int32_t* seg, int b, int kk, int L) {
  const int32_t* p = seg + (size_t)b * L;
  if ((L & 3) == 0 && kk + 3 < L) return *(const int4*)(p + kk);
  int4 r;
  r.x = kk < L ? p[kk] : 0;
  r.y = kk + 1 < L ? p[kk + 1] : 0;
  r.z = kk + 2 < L ? p[kk + 2] : 0;
  r.w = kk + 3 < L ? p[kk + 3] : 0;
  return r;
}

// Bias for this lane's query row at 4 consecutive keys starting at kk.
template <bool VEC>
__device__ __forceinline__ f32x4 load_bias4(const float* row, int kk, int Lk) {
  if (VEC && kk + 3 < Lk) return *(const f32x4*)(row + kk);
  f32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = (kk + j < Lk) ? row[kk + j] : 0.f;
  return r;
}

// bf16 K/V tile layout: BK keys per tile, row-major [key][dim] rows of D*2
// bytes, 16-byte chunks XOR-swizzled per row.  K: a ds_read_b128 fragment has
// lane l read chunk 2*st + l/32 of row l%32, and gfx950's LDS serves lanes
// 0-7 with 24-31 and 8-15 with 16-23 in one cycle (64 banks of 4 bytes), so
// rows r < 8 and r + 24 (or r + 8 and r + 16) must take different 16-byte
// bank groups: chunk ^ (row & 15) at D = 128 (whole bank lines); at D = 64,
// where odd rows start half a line later, chunk ^ ((row & 6) | ((row >> 3) & 1))
// (with row & 7 the two halves of each cycle met in one bank group).  V:
// chunk ^ f(row) chosen so a transposing read of 4 rows x 32 bytes per 16
// lanes hits distinct banks.
template <int D, int BK_ = 64>
struct Bf16Tile {
  static constexpr int BK = BK_;            // keys per tile
  static constexpr int ROWB = D * 2;        // bytes per K/V row
  static constexpr int NC = D / 8;          // 16-byte chunks per row
  static constexpr int TILE_B = BK * ROWB;  // bytes of one K (or V) tile
  static constexpr int STAGE_B = 2 * TILE_B;
  static constexpr int RPI = 64 / NC;       // rows per 1 KiB buffer->LDS load
  static constexpr int NLD = (BK / 4) / RPI;  // loads per wave per tensor per tile
  __device__ static int swz_k(int r) { return NC >= 16 ? (r & 15) : ((r & 6) | ((r >> 3) & 1)); }
  __device__ static int swz_v(int r) {
    return D == 128 ? 4 * (r & 3) + 2 * ((r >> 1) & 1) : 4 * ((r >> 1) & 1) + 2 * (r & 1);
  }
};

// Host: checks the C-ABI modifier block and fills a.m / a.ext; returns a
// PJX_* status (message set on error).
int lower_score_mods(const pjx_score_mods* mods, FlashArgs& a, const char* who);

// Launches the bf16 dense-bias kernel (flash_bias_ring.hip); returns a PJX_*
// status.
int launch_flash_bias_ring(int head_dim, const FlashArgs& a, hipStream_t stream);

// Arguments of the wide-head backward kernels (flash_wide_bwd.hip).
struct WideBwdArgs {
  FlashArgs f;        // q, k, v, o (forward output), lse, masks, bias, sizes; f.dv = DV
  const void* dout;   // dO [B, Lq, Hq, DV]
  float* delta;       // workspace [B, Hq, Lq]
  float* lse2;        // workspace [B, Hq, Lq]: lse * log2e
  void* dq;           // [B, Lq, Hq, D]
  void* dk;           // [B, Lk, Hkv, D]; with the shared latent dC [B, Lk, D]
  void* dv;           // [B, Lk, Hkv, DV] (separate K / V only)
  float* dbias;       // [B, Hq, Lq, Lk] fp32 dL/d(bias) or null
  float* part;        // [nsplit][B][Lk][Hkv][D (+ DV)] fp32 partials when nsplit > 1
  int nsplit;         // query-head groups per KV head in the dK/dV kernel
  // The rounded dS kept between the dK/dV and dQ kernels (the dS route of
  // flash_wide_bwd.hip), or null: per query head, blocks of 32 queries x 16
  // keys (1 KiB), ds_nq32 x ds_nk16 of them ([query block][key block]).
  uint16_t* ds;
  int ds_nq32, ds_nk16;
};

// The wide backward's dS blocks (the dS route) for these sizes: 32-query
// blocks over the queries rounded up to the dQ kernel's 64-row tiles, 16-key
// blocks over the keys rounded up to the dK/dV kernel's 64-key tiles.
inline int64_t wide_bwd_ds_nq32(int64_t Lq) { return 2 * ((Lq + 63) / 64); }
inline int64_t wide_bwd_ds_nk16(int64_t Lk) { return 4 * ((Lk + 63) / 64); }
size_t wide_bwd_ds_bytes(int64_t B, int64_t Hq, int64_t Lq, int64_t Lk);

// Runs the wide backward (dQ, then dK/dV or the latent's dC, then the partial
// sum when nsplit > 1; with dq_only the dQ kernel alone, which also writes
// delta and lse*log2e; with ba.ds at D = 256 and no bias or extended masks,
// the dS route: delta, dK/dV storing dS, dQ from dS); returns a PJX_* status.
int run_wide_bwd(WideBwdArgs& ba, int D, int DV, bool shared, hipStream_t s, const char* who,
                 bool dq_only = false);
// Byte offset of the dS blocks in a dS-route workspace whose leading part
// (delta, lse*log2e, partials) takes `lead` bytes.
inline size_t wide_bwd_ds_offset(size_t lead) { return (lead + 255) & ~(size_t)255; }

// Wide-head bf16 forward kernels (flash_wide.hip): D = 256 with separate K/V,
// and the absorbed latent (K = V, rank 512 / 576, output width a.dv).
int launch_flash_wide256(FlashArgs& a, hipStream_t stream);
int launch_mla_wide(FlashArgs& a, int rank, hipStream_t stream);

}  // namespace pjx

namespace pjx {

// Extended masks and modifiers on one key tile in the S^T layout (lane =
// query g.qi; register r of block kb = key k0 + kb*32 + 8*(r/4) + 4*half +
// r%4).  For every raw score q.k, emit(kb, r, x, g) receives the modified
// score x (-inf where masked) and the modifier's derivative g.
template <int NKB, bool BIAS, bool SOFTCAP, typename Emit>
__device__ __forceinline__ void ext_scores_sT_t(const FlashArgs& a, const BlockGeom& g,
                                              const ExtRows& er, const f32x16* s, int k0, int half,
                                              const float* brow, bool row_in, Emit emit) {
  const bool bias_vec = (a.Lk & 3) == 0;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int kk = k0 + kb * 32 + 8 * gq + 4 * half;
      f32x4 bv = {0.f, 0.f, 0.f, 0.f};
      if constexpr (BIAS) {
        if (row_in) bv = bias_vec ? load_bias4<true>(brow, kk, a.Lk) : load_bias4<false>(brow, kk, a.Lk);
      }
      int4 sg = {0, 0, 0, 0};
      if (a.m.seg_k) sg = seg4(a.m.seg_k, g.b, kk, a.Lk);
      const int sgv[4] = {sg.x, sg.y, sg.z, sg.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * gq + j, kj = kk + j;
        float gg;
        const float x = modify_score<SOFTCAP>(a.m, er.hm, s[kb][r] * a.scale, bv[j], g.qi, kj, gg);
        const bool keep = kj >= er.lo && kj <= er.hi &&
                          (!a.m.seg_q || (a.m.seg_lt ? kj < er.segq : sgv[j] == er.segq));
        emit(kb, r, keep ? x : -INFINITY, gg);
      }
      // one group of 4 keys at a time: keeps the loads and temporaries of
      // the groups from piling up in registers
      __builtin_amdgcn_sched_barrier(0);
    }
}

// Interval masks only (the positional masks; no segment ids or modifiers)
// in the S^T layout: scores outside this row's key interval become -inf.
// Tiles inside the interval of every row of the wave are left alone.
template <int NKB>
__device__ __forceinline__ void ext_mask_sT(const BlockGeom& g, const ExtRows& er, f32x16* s, int k0,
                                            int half) {
  constexpr int BK = NKB * 32;
  if (k0 >= er.lo_last && k0 + BK - 1 <= er.hi_first && g.qw + 31 < g.q_hi) return;
  const int base = k0 + 4 * half;
  const int lo = er.lo - base, hi = er.hi - base;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int o = kb * 32 + 8 * (r >> 2) + (r & 3);
      if (o < lo || o > hi) s[kb][r] = -INFINITY;
    }
}

// The same in the S layout (lane = key with query rows [qlo, qhi]; register
// r = query qs0 + 8*(r/4) + 4*half + r%4); `need` false skips the step.
__device__ __forceinline__ void ext_mask_S(f32x16& s, int qs0, int half, int qlo, int qhi, bool need) {
  if (!need) return;
  const int base = qs0 + 4 * half;
  const int lo = qlo - base, hi = qhi - base;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int o = 8 * (r >> 2) + (r & 3);
    if (o < lo || o > hi) s[r] = -INFINITY;
  }
}

// The same in the S layout of the dK/dV kernels (lane = key `key`, register
// r = query qs0 + 8*(r/4) + 4*half + r%4); [qlo, qhi] are the rows that see
// `key`, segk its segment id, bbase the bias slice of (b, h).
// emit(r, x, g) as above.
template <bool BIAS, bool SOFTCAP, typename Emit>
__device__ __forceinline__ void ext_scores_S_t(const FlashArgs& a, int b, const HeadMods& hm, int key,
                                             int qlo, int qhi, int segk, const f32x16& s, int qs0,
                                             int half, const float* bbase, Emit emit) {
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) {
    const int q4 = qs0 + 8 * gq + 4 * half;
    int4 sg = {0, 0, 0, 0};
    if (a.m.seg_q) sg = seg4(a.m.seg_q, b, q4, a.Lq);
    const int sgv[4] = {sg.x, sg.y, sg.z, sg.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 4 * gq + j, qr = q4 + j;
      float bv = 0.f;
      if constexpr (BIAS) bv = (qr < a.Lq && key < a.Lk) ? bbase[(size_t)qr * a.Lk + key] : 0.f;
      float gg;
      const float x = modify_score<SOFTCAP>(a.m, hm, s[r] * a.scale, bv, qr, key, gg);
      const bool keep = qr >= qlo && qr <= qhi &&
                        (!a.m.seg_q || (a.m.seg_lt ? key < sgv[j] : sgv[j] == segk));
      emit(r, keep ? x : -INFINITY, gg);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The soft cap (two transcendentals per score) is chosen once per tile.
template <int NKB, bool BIAS, typename Emit>
__device__ __forceinline__ void ext_scores_sT(const FlashArgs& a, const BlockGeom& g,
                                              const ExtRows& er, const f32x16* s, int k0, int half,
                                              const float* brow, bool row_in, Emit emit) {
  if (a.m.softcap > 0.f)
    ext_scores_sT_t<NKB, BIAS, true>(a, g, er, s, k0, half, brow, row_in, emit);
  else
    ext_scores_sT_t<NKB, BIAS, false>(a, g, er, s, k0, half, brow, row_in, emit);
}

template <bool BIAS, typename Emit>
__device__ __forceinline__ void ext_scores_S(const FlashArgs& a, int b, const HeadMods& hm, int key,
                                             int qlo, int qhi, int segk, const f32x16& s, int qs0,
                                             int half, const float* bbase, Emit emit) {
  if (a.m.softcap > 0.f)
    ext_scores_S_t<BIAS, true>(a, b, hm, key, qlo, qhi, segk, s, qs0, half, bbase, emit);
  else
    ext_scores_S_t<BIAS, false>(a, b, hm, key, qlo, qhi, segk, s, qs0, half, bbase, emit);
}

}  // namespace pjx
