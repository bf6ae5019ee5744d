// Flash-attention backward for gfx950 (bf16, fp16 or fp32 inputs, fp32 accumulation).
//
// Replaces the Pallas backward of probjax's `mha`:
//   _preprocess_backward_kernel (probjax/nn/pallas_kernels/kernels/attention.py:853-867)
//   mha_backward_kernel         (:909-1160; scan #1 dK/dV :989-1052, scan #2 dQ :1089-1150)
//   _mha_backward_raw           (:3505-3560; GQA group sums :2123-2128)
// with the math of those kernels:
//   delta = sum_d o * do;  p = exp2(s * log2e - lse * log2e);  dp = do . v^T
//   ds = p * (dp - delta) * sm_scale
//   dv = sum_q r(p)^T do,  dk = sum_q r(ds)^T q,  dq = sum_k r(ds) k,
// r() rounding to the input's 16-bit format (bf16 or fp16; none in fp32).
// s is the forward's score: sm_scale * q.k [+ bias], masked keys excluded.
// lse is the forward's natural-log residual (+inf for rows without a valid
// key: p = 0 there, so those rows contribute nothing).
//
// Two kernels on the caller's stream:
//   flash_bwd_dq_kernel   -- one workgroup per (128-query tile, batch, head),
//     as the forward: K/V tiles of 64 keys stream HBM -> LDS; S^T = K Q^T and
//     dP^T = V dO^T with keys as MFMA rows, so each lane holds one query's
//     column and its lse / delta are one register each; dQ^T += K^T dS^T with
//     K^T read by transposing LDS reads.  It also computes delta for its rows
//     (o and dO are read once, for dO^T) and writes delta * sm_scale and
//     lse*log2e to the workspace for the second kernel, which then forms
//     dS = P (dP sm_scale - delta sm_scale) with one fma and one multiply.
//   flash_bwd_dkdv_kernel -- one workgroup per (128-key tile, batch, KV head),
//     each wave owns 32 keys whose K^T and V^T stay in registers; Q and dO
//     tiles of 64 queries of every query head of the group stream through
//     LDS.  S = Q K^T and dP = dO V^T put queries on the MFMA rows, so P and
//     dS in registers are directly the B operands of dV^T += dO^T P and
//     dK^T += Q^T dS (dO^T and Q^T by transposing LDS reads).  The group's
//     query heads accumulate in fp32 before the single rounding to 16 bits.
//
// D = 64 and 128 run both kernels at two waves per SIMD.  At D = 256 (16-bit,
// no extended masks) dQ comes from the wide-head kernel of flash_wide_bwd.hip
// and dK/dV from flash_bwd_dkdv_kernel at one wave per SIMD, the faster pair
// on the causal 4096-token case; with extended masks both come from the
// wide-head kernels.
//
// LDS tiles (both kernels) are row-major [row][dim] with 16-byte chunks
// XOR-swizzled so that both reads of a tile are free of bank conflicts: the
// 16-byte reads of one chunk column over 16 consecutive rows, and the
// transposing 8-byte reads of 4 aligned rows x 4 consecutive chunks.
#pragma once

#include "flash_common.h"

namespace pjx {

struct FlashBwdArgs {
  FlashArgs f;        // q, k, v, o (forward output), lse, masks, bias, sizes
  const void* dout;   // dO [B, Lq, Hq, D]
  float* delta;       // workspace [B, Hq, Lq]
  float* lse2;        // workspace [B, Hq, Lq]: lse * log2e
  void* dq;
  void* dk;
  void* dv;
  float* dbias;       // [B, Hq, Lq, Lk] fp32 dL/d(bias): P (dP - delta) per score, or null
};

constexpr int kBKV = 128;  // keys per dK/dV workgroup (32 per wave)
constexpr int kBQs = 64;   // queries per dK/dV LDS stage

template <int D>
struct BwdTile {
  static constexpr int ROWS = 64;            // rows per tile
  static constexpr int ROWB = D * 2;         // bytes per row
  static constexpr int NC = D / 8;           // 16-byte chunks per row
  static constexpr int TILE_B = ROWS * ROWB;
  static constexpr int RPI = 64 / NC;        // rows per 1 KiB wave load
  static constexpr int NLD = (ROWS / 4) / RPI;  // loads per wave per tensor per tile
  // Bijective over any 16 consecutive rows (16-byte column reads), and the
  // 4 rows of an aligned group differ in the chunk bits above the 4-chunk
  // block of a transposing read (D=128, 256: bits 3:2 of the chunk within its
  // bank line; D=64 with two rows per bank line: bit 2 between rows of equal
  // parity).
  __device__ static int swz(int r) {
    return D >= 128 ? (((r & 3) << 2) | ((r >> 2) & 3)) : ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
  }
};

// Per-lane LDS byte offsets of a tile's two read patterns.
template <int D>
struct BwdOffsets {
  using T = BwdTile<D>;
  uint32_t row[D / 16];   // A = X[row][dim]: row `col` of a 32-row block, dims 16*s + 8*half
  uint32_t tlo[D / 32];   // A = X^T: transposing reads, rows 4*half + s16/4 of a 16-row step
  uint32_t thi[D / 32];   // ... and rows 8 + 4*half + s16/4
  // base: byte offset added to every offset (a wave group's stage)
  __device__ void init(int lane, uint32_t base = 0) {
    const int col = lane & 31, half = lane >> 5;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) row[s] = base + col * T::ROWB + 16 * ((2 * s + half) ^ T::swz(col));
    const int s16 = lane & 15, grp = lane >> 4;
    const int r = 4 * half + s16 / 4;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int chunk = 4 * db + 2 * (grp & 1) + ((s16 & 3) >> 1);
      tlo[db] = base + r * T::ROWB + 16 * (chunk ^ T::swz(r)) + 8 * (s16 & 1);
      thi[db] = base + (r + 8) * T::ROWB + 16 * (chunk ^ T::swz(r + 8)) + 8 * (s16 & 1);
    }
  }
};

// A operand X^T (dims 32*db.., 16 rows starting at row0 in slot order
// 8*(j/4) + 4*half + j%4) from a row-major tile.
template <typename E, int D>
__device__ __forceinline__ typename E::v8 read_t(const unsigned char* tile, int row0, uint32_t lo, uint32_t hi) {
  const unsigned char* p = tile + row0 * BwdTile<D>::ROWB;
  const u32x2 a = lds_read_tr16(p + lo);
  const u32x2 b = lds_read_tr16(p + hi);
  const u32x4 v = {a[0], a[1], b[0], b[1]};
  return E::as8(v);
}

// Registers of a 32x32 C block as the B operand of the next product:
// k-step c (16 rows) holds registers 8c .. 8c+7, rounded to the 16-bit format.
template <typename E>
__device__ __forceinline__ typename E::v8 pack_step(const f32x16& x, int c) {
  u32x4 pk;
#pragma unroll
  for (int j = 0; j < 4; ++j) pk[j] = E::pack2(x[8 * c + 2 * j], x[8 * c + 2 * j + 1]);
  return E::as8(pk);
}

// dL/d(bias) of one key tile in the S^T layout (lane = query g.qi, register
// r of block kb = key k0 + kb*32 + 8*(r/4) + 4*half + r%4): 4 consecutive
// keys per register group go out as one 16-byte store.  Tiles the kernel
// skips (fully masked) are left as the caller's zeros.
template <int NKB>
__device__ __forceinline__ void store_dbias(const FlashBwdArgs& ba, const BlockGeom& g,
                                            const f32x16* dbv, int k0, int half, bool row_in) {
  const FlashArgs& a = ba.f;
  if (!row_in) return;
  float* row = ba.dbias + (((size_t)g.b * a.Hq + g.h) * a.Lq + g.qi) * a.Lk;
  const bool vec = (a.Lk & 3) == 0;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int kk = k0 + kb * 32 + 8 * gq + 4 * half;
      if (vec && kk + 3 < a.Lk) {
        *(f32x4*)(row + kk) = f32x4{dbv[kb][4 * gq], dbv[kb][4 * gq + 1], dbv[kb][4 * gq + 2], dbv[kb][4 * gq + 3]};
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (kk + j < a.Lk) row[kk + j] = dbv[kb][4 * gq + j];
      }
    }
}

// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// dQ (and delta): one workgroup per (128-query tile, batch, head).  NG = 2
// (small grids): 8 waves, two groups of 4 over the same 128 queries; group j
// takes the key tiles t with t % 2 == j through its own 2-stage ring, and at
// the end group 1 adds its dQ sums into group 0's through LDS.
// ---------------------------------------------------------------------------
template <typename E, int D, int BIAS, int EXT, int NG = 1>
__global__ __launch_bounds__(NG * kThreads, (D <= 128 ? 2 : 1)) void flash_bwd_dq_kernel(FlashBwdArgs ba) {
  // BIAS: 0 none, 1 dense bias, 2 dense bias and its gradient (ba.dbias)
  constexpr bool HB = BIAS != 0, DB = BIAS == 2;
  const FlashArgs& a = ba.f;
  using T = BwdTile<D>;
  constexpr int BK = T::ROWS, ROWB = T::ROWB, TILE_B = T::TILE_B;
  constexpr int STAGE_B = 2 * TILE_B;
  static_assert(NG == 1 || NG == 2 && EXT == 0, "one group, or two without extended masks");
  __shared__ __attribute__((aligned(1024))) unsigned char smem0[NG * STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char smem1[NG * STAGE_B];

  BlockGeom g = block_geom(a);
  if constexpr (EXT > 0) ext_block_range(a, g, BK);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w8 = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gi = NG > 1 ? w8 >> 2 : 0;   // group: the key tiles t with t % NG == gi
  const int w = NG > 1 ? (w8 & 3) : w8;  // wave within the group: rows 32w .. of the q tile
  if constexpr (NG > 1) {
    g.qw = g.q0 + 32 * w;
    g.qi = g.qw + (tid & 31);
  }
  g.qw = __builtin_amdgcn_readfirstlane(g.qw);
  unsigned char* const st0 = smem0 + gi * STAGE_B;  // this group's stages
  unsigned char* const st1 = smem1 + gi * STAGE_B;
  const int col = lane & 31, half = lane >> 5;
  const uint32_t rowstride = (uint32_t)a.Hkv * D * 2;
  const unsigned char* Kb = (const unsigned char*)a.k + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * ROWB;
  const unsigned char* Vb = (const unsigned char*)a.v + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * ROWB;
  const bool row_in = g.qi < a.Lq;
  const bool row_ok = g.qi < g.q_hi;

  // Q^T and dO^T as B operands (lane: query `col`, dims 16*s + 8*half + [0,8)),
  // and delta = sum_d o*do of this query over both halves.
  typename E::v8 qf[D / 16], dof[D / 16];
  float dsum = 0.f;
  {
    const size_t roff = ((size_t)(g.b * a.Lq + (row_in ? g.qi : 0)) * a.Hq + g.h) * D;
    const uint16_t* qrow = (const uint16_t*)a.q + roff;
    const uint16_t* drow = (const uint16_t*)ba.dout + roff;
    const uint16_t* orow = (const uint16_t*)a.o + roff;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      u32x4 rq = {0u, 0u, 0u, 0u}, rd = rq, ro = rq;
      if (row_in) {
        rq = *(const u32x4*)(qrow + 16 * s + 8 * half);
        rd = *(const u32x4*)(drow + 16 * s + 8 * half);
        ro = *(const u32x4*)(orow + 16 * s + 8 * half);
      }
      qf[s] = E::as8(rq);
      dof[s] = E::as8(rd);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dsum = fmaf(E::lo(ro[j]), E::lo(rd[j]), fmaf(E::hi(ro[j]), E::hi(rd[j]), dsum));
    }
  }
  const float delta = xor32_sum(dsum);
  const float dsc = delta * a.scale;  // the workspace holds delta * sm_scale
  float lse2 = 0.f;
  const size_t lidx = ((size_t)g.b * a.Hq + g.h) * a.Lq + g.qi;
  if (row_in) {
    lse2 = a.lse[lidx] * kLog2e;
    if (half == 0 && gi == 0) {
      ba.delta[lidx] = dsc;
      ba.lse2[lidx] = lse2;
    }
  }
  const float* brow = nullptr;
  if constexpr (HB) {
    brow = a.bias + (size_t)g.b * a.bias_bstride + (size_t)g.h * a.bias_hstride +
           (size_t)(row_in ? g.qi : 0) * a.Lk;
  }
  const bool bias_vec = (a.Lk & 3) == 0;
  const float cx = (HB || EXT == 2) ? kLog2e : a.scale * kLog2e;
  ExtRows er;
  if constexpr (EXT > 0) er = ext_rows(a, g);

  uint32_t voff[T::NLD];
#pragma unroll
  for (int j = 0; j < T::NLD; ++j) {
    const int r = 16 * w + T::RPI * j + lane / T::NC, slot = lane % T::NC;
    voff[j] = r * rowstride + 16 * (slot ^ T::swz(r));
  }
  BwdOffsets<D> off;
  off.init(lane, gi * STAGE_B);  // fragment reads address the group's stage from smem0 / smem1

  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16{};

  const int t_begin = g.kv_begin / BK;
  const int n_tiles = max((g.kv_stop + BK - 1) / BK - t_begin, 0);
  const int q_last_w = g.qw + 31;

  auto issue = [&](int t, unsigned char* ks) {
    const int k0 = (t_begin + t) * BK;
    const int nvalid = min(BK, g.kv_stop - k0);
    const uint32_t bytes = (uint32_t)(nvalid - 1) * rowstride + ROWB;
    const rsrc_t rk = make_rsrc(Kb + (size_t)k0 * rowstride, bytes);
    const rsrc_t rv = make_rsrc(Vb + (size_t)k0 * rowstride, bytes);
#pragma unroll
    for (int j = 0; j < T::NLD; ++j) {
      const int r0 = 16 * w + T::RPI * j;
      buffer_load_lds16(rk, ks + r0 * ROWB, voff[j]);
      buffer_load_lds16(rv, ks + TILE_B + r0 * ROWB, voff[j]);
    }
  };

  auto compute = [&](int t, const unsigned char* ks) {
    const int k0 = (t_begin + t) * BK;
    if constexpr (EXT > 0) {
      if (!er.any || k0 > er.hi_last || k0 + BK - 1 < er.lo_first) return;
    } else {
      if (a.causal && k0 > q_last_w) return;  // tile above this wave's diagonal
    }
    const unsigned char* vs = ks + TILE_B;

    // S^T[key][query] = K Q^T and dP^T = V dO^T; register r of block kb holds
    // key k0 + kb*32 + 8*(r/4) + 4*half + r%4 of query `col`.
    f32x16 s[BK / 32], dp[BK / 32];
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb) {
      s[kb] = f32x16{};
      dp[kb] = f32x16{};
#pragma unroll
      for (int st = 0; st < D / 16; ++st) {
        const typename E::v8 kf = E::as8(*(const u32x4*)(ks + kb * 32 * ROWB + off.row[st]));
        s[kb] = E::mma32(kf, qf[st], s[kb]);
      }
#pragma unroll
      for (int st = 0; st < D / 16; ++st) {
        const typename E::v8 vf = E::as8(*(const u32x4*)(vs + kb * 32 * ROWB + off.row[st]));
        dp[kb] = E::mma32(vf, dof[st], dp[kb]);
      }
    }
    PJX_SCHED_LDS_READS_AHEAD(2 * (D / 16) * (BK / 32), 3, 1);  // K / V fragments 3 MFMAs ahead
    f32x16 dbv[DB ? BK / 32 : 1];  // dL/d(bias) = P (dP - delta), kept for the store
    if constexpr (EXT == 2) {
      // modified scores, masks, P and dS = P (dP - delta) * scale * f'(s)
      ext_scores_sT<BK / 32, HB>(a, g, er, s, k0, half, brow, row_in,
                                 [&](int kb, int r, float x, float gg) {
                                   const float p = fast_exp2(fmaf(x, cx, -lse2));
                                   const float t = p * (dp[kb][r] - delta);
                                   if constexpr (DB) dbv[kb][r] = t;
                                   s[kb][r] = t * a.scale * gg;
                                 });
    } else {
    if constexpr (HB) {
#pragma unroll
      for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int kk = k0 + kb * 32 + 8 * gq + 4 * half;
          f32x4 bv = {0.f, 0.f, 0.f, 0.f};
          if (row_in) bv = bias_vec ? load_bias4<true>(brow, kk, a.Lk) : load_bias4<false>(brow, kk, a.Lk);
#pragma unroll
          for (int j = 0; j < 4; ++j) s[kb][4 * gq + j] = fmaf(s[kb][4 * gq + j], a.scale, bv[j]);
        }
    }
    if constexpr (EXT == 1) ext_mask_sT<BK / 32>(g, er, s, k0, half);
    const bool need_mask = EXT == 0 && ((k0 + BK > g.kv_end) || (a.causal && k0 + BK - 1 > g.qw) ||
                                        (g.qw + 31 >= g.q_hi));
    if (need_mask) {
      const int base = k0 + 4 * half;
      int lim = g.kv_end - 1 - base;
      if (a.causal) lim = min(lim, g.qi - base);
      if (!row_ok) lim = -1;
#pragma unroll
      for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kb * 32 + 8 * (r >> 2) + (r & 3) > lim) s[kb][r] = -INFINITY;
    }
    // dS^T = P^T (dP^T - delta) * scale, rounded to 16 bits as the B operand.
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(s[kb][r], cx, -lse2));
        if constexpr (DB) {
          const float t = p * (dp[kb][r] - delta);
          dbv[kb][r] = t;
          s[kb][r] = t * a.scale;
        } else {
          s[kb][r] = p * fmaf(dp[kb][r], a.scale, -dsc);  // p (dp - delta) scale
        }
      }
    }
    if constexpr (DB) store_dbias<BK / 32>(ba, g, dbv, k0, half, row_in);
    typename E::v8 dsf[BK / 16];
#pragma unroll
    for (int c = 0; c < BK / 16; ++c) dsf[c] = pack_step<E>(s[c >> 1], c & 1);
    // dQ^T[d][query] += K^T dS^T
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int c = 0; c < BK / 16; ++c)
        acc[db] = E::mma32(read_t<E, D>(ks, 16 * c, off.tlo[db], off.thi[db]), dsf[c], acc[db]);
  };

  // this group's tiles NG*s + gi: n_loc of them; n_steps (the same for every
  // group) keeps the barriers in step
  const int n_loc = (n_tiles - gi + NG - 1) / NG;
  const int n_steps = (n_tiles + NG - 1) / NG;
  if (n_loc > 0) issue(gi, st0);
  for (int s = 0; s < n_steps; s += 2) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (s + 1 < n_loc) issue(NG * (s + 1) + gi, st1);
    if (s < n_loc) compute(NG * s + gi, smem0);
    if (s + 1 >= n_steps) break;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (s + 2 < n_loc) issue(NG * (s + 2) + gi, st0);
    if (s + 1 < n_loc) compute(NG * (s + 1) + gi, smem1);
  }
  if constexpr (NG > 1) {
    // Group 1 hands its dQ^T sums to group 0 through LDS, lane by lane in the
    // same register layout: 16-byte quads [D/32 * 4][4 waves][64 lanes].
    static_assert((D / 32) * 4 * 256 * 16 <= NG * STAGE_B, "hand-off fits");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // every wave is done with the rings
    f32x4* xq = (f32x4*)smem0 + w * 64 + lane;
    if (gi == 1) {
#pragma unroll
      for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int r = 0; r < 16; r += 4)
          xq[(4 * i + r / 4) * 256] = f32x4{acc[i][r], acc[i][r + 1], acc[i][r + 2], acc[i][r + 3]};
    }
    __syncthreads();
    if (gi == 1) return;
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        const f32x4 q1 = xq[(4 * i + r / 4) * 256];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][r + j] += q1[j];
      }
  }

  if (row_in) {
    uint16_t* drow = (uint16_t*)ba.dq + ((size_t)(g.b * a.Lq + g.qi) * a.Hq + g.h) * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        u32x2 pk;
        pk[0] = E::pack2(acc[db][4 * gq], acc[db][4 * gq + 1]);
        pk[1] = E::pack2(acc[db][4 * gq + 2], acc[db][4 * gq + 3]);
        *(u32x2*)(drow + db * 32 + 8 * gq + 4 * half) = pk;
      }
  }
}

// ---------------------------------------------------------------------------
// dK, dV: one workgroup per (128-key tile, batch, KV head).  NG = 2 (small
// grids): 8 waves, two groups of 4 over the same 128 keys; group j takes the
// (query tile, head) steps t with t % 2 == j through its own 2-stage ring, and
// at the end group 1 adds its dK / dV sums into group 0's through LDS.
// ---------------------------------------------------------------------------
template <typename E, int D, bool BIAS, int EXT, int NG = 1>
__global__ __launch_bounds__(NG * kThreads, (D <= 128 ? 2 : 1)) void flash_bwd_dkdv_kernel(FlashBwdArgs ba) {
  const FlashArgs& a = ba.f;
  using T = BwdTile<D>;
  constexpr int ROWB = T::ROWB, TILE_B = T::TILE_B;
  static_assert(T::ROWS == kBQs, "one Q / dO tile per stage");
  // Per stage: Q tile, dO tile, then each wave's own copy of the stage's
  // lse*log2e and delta * sm_scale (64 floats each).
  constexpr int SMALL_B = 2 * kBQs * 4;
  constexpr int STAGE_B = 2 * TILE_B + 4 * SMALL_B;
  static_assert(NG == 1 || NG == 2, "one or two groups");
  __shared__ __attribute__((aligned(1024))) unsigned char smem0[NG * STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char smem1[NG * STAGE_B];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w8 = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gi = NG > 1 ? w8 >> 2 : 0;   // group: the steps t with t % NG == gi
  const int w = NG > 1 ? (w8 & 3) : w8;  // wave within the group: keys 32w .. of the tile
  unsigned char* const st0 = smem0 + gi * STAGE_B;  // this group's stages
  unsigned char* const st1 = smem1 + gi * STAGE_B;
  const int col = lane & 31, half = lane >> 5;
  const int BH = a.B * a.Hkv;
  const int bh = blockIdx.x % BH;
  const int k0 = (blockIdx.x / BH) * kBKV;
  const int b = bh / a.Hkv, hkv = bh % a.Hkv;
  const int G = a.Hq / a.Hkv;
  const int kw = k0 + 32 * w;
  const int key = kw + col;
  int kv_end = min(a.Lk, a.kv_valid);
  if (a.kv_lengths) kv_end = min(kv_end, max(a.kv_lengths[b], 0));
  const int q_hi = min(a.Lq, a.q_valid);
  // Queries that can see a key of this tile: causal rows start at k0; with
  // extended masks the rows [qlo(k0), qhi(last key)] (both monotone).
  int q_begin = a.causal ? (k0 / kBQs) * kBQs : 0;
  int q_end = q_hi;
  int qlo = 0, qhi = q_hi - 1, wq_first = 0, wq_last = q_hi - 1, segk = 0;
  int qhi_first = q_hi - 1, qlo_last = 0;  // rows seen by every key of the wave: [qlo_last, qhi_first]
  if constexpr (EXT > 0) {
    q_end = q_begin = 0;
    if (k0 < kv_end) {
      int a0, a1, b0, b1;
      key_bounds(a.m, a.causal, b, kv_end, q_hi, k0, a0, a1);
      key_bounds(a.m, a.causal, b, kv_end, q_hi, min(k0 + kBKV, kv_end) - 1, b0, b1);
      q_begin = max(a0, 0);
      q_end = b1 + 1;
    }
    key_bounds(a.m, a.causal, b, kv_end, q_hi, key, qlo, qhi);
    if (kw < kv_end) {
      key_bounds(a.m, a.causal, b, kv_end, q_hi, kw, wq_first, qhi_first);
      key_bounds(a.m, a.causal, b, kv_end, q_hi, min(kw + 32, kv_end) - 1, qlo_last, wq_last);
    }
    if (a.m.seg_k && key < a.Lk) segk = a.m.seg_k[(size_t)b * a.Lk + key];
  }
  const int n_qt = (k0 < kv_end && q_end > q_begin) ? (q_end - q_begin + kBQs - 1) / kBQs : 0;
  const int n_tiles = G * n_qt;

  // K^T and V^T as B operands: lane holds key `key`, dims 16*s + 8*half + [0,8).
  typename E::v8 kf[D / 16], vf[D / 16];
  {
    const bool kin = key < a.Lk;
    const size_t koff = ((size_t)(b * a.Lk + (kin ? key : 0)) * a.Hkv + hkv) * D;
    const uint16_t* krow = (const uint16_t*)a.k + koff;
    const uint16_t* vrow = (const uint16_t*)a.v + koff;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      u32x4 rk = {0u, 0u, 0u, 0u}, rv = rk;
      if (kin) {
        rk = *(const u32x4*)(krow + 16 * s + 8 * half);
        rv = *(const u32x4*)(vrow + 16 * s + 8 * half);
      }
      kf[s] = E::as8(rk);
      vf[s] = E::as8(rv);
    }
  }
  const float cx = (BIAS || EXT == 2) ? kLog2e : a.scale * kLog2e;
  const uint32_t rowstride = (uint32_t)a.Hq * D * 2;

  uint32_t voff[T::NLD];
#pragma unroll
  for (int j = 0; j < T::NLD; ++j) {
    const int r = 16 * w + T::RPI * j + lane / T::NC, slot = lane % T::NC;
    voff[j] = r * rowstride + 16 * (slot ^ T::swz(r));
  }
  BwdOffsets<D> off;
  off.init(lane, gi * STAGE_B);  // fragment reads address the group's stage from smem0 / smem1

  f32x16 acck[D / 32], accv[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    acck[i] = f32x16{};
    accv[i] = f32x16{};
  }

  // Query tiles last to first, the group's heads innermost: the workgroups of
  // one KV head's key blocks (same XCD, running together) then stream the same
  // Q / dO tile at the same time, so all but the first read it from L2
  // (causal: each starts at the sequence's end and stops at its own keys).
  auto tile_head = [&](int t) { return hkv * G + t % G; };
  auto tile_q0 = [&](int t) { return q_begin + (n_qt - 1 - t / G) * kBQs; };

  auto issue = [&](int t, unsigned char* st) {
    const int h = tile_head(t), q0 = tile_q0(t);
    const int nvalid = max(min(kBQs, a.Lq - q0), 1);
    const uint32_t bytes = (uint32_t)(nvalid - 1) * rowstride + ROWB;
    const size_t roff = ((size_t)(b * a.Lq + q0) * a.Hq + h) * ROWB;
    const rsrc_t rq = make_rsrc((const unsigned char*)a.q + roff, bytes);
    const rsrc_t rd = make_rsrc((const unsigned char*)ba.dout + roff, bytes);
#pragma unroll
    for (int j = 0; j < T::NLD; ++j) {
      const int r0 = 16 * w + T::RPI * j;
      buffer_load_lds16(rq, st + r0 * ROWB, voff[j]);
      buffer_load_lds16(rd, st + TILE_B + r0 * ROWB, voff[j]);
    }
    const size_t loff = ((size_t)b * a.Hq + h) * a.Lq + q0;
    const rsrc_t rl = make_rsrc(ba.lse2 + loff, (uint32_t)nvalid * 4);
    const rsrc_t rdl = make_rsrc(ba.delta + loff, (uint32_t)nvalid * 4);
    unsigned char* small = st + 2 * TILE_B + w * SMALL_B;
    buffer_load_lds4(rl, small, 4 * lane);
    buffer_load_lds4(rdl, small + kBQs * 4, 4 * lane);
  };

  auto compute = [&](int t, const unsigned char* st) {
    const int h = tile_head(t), q0 = tile_q0(t);
    const unsigned char* qs = st;
    const unsigned char* dos = st + TILE_B;
    const float* lsm = (const float*)(st + gi * STAGE_B + 2 * TILE_B + w * SMALL_B);
    const float* dlm = lsm + kBQs;
    const float* bbase = nullptr;
    if constexpr (BIAS) bbase = a.bias + (size_t)b * a.bias_bstride + (size_t)h * a.bias_hstride;
#pragma unroll
    for (int qb = 0; qb < kBQs / 32; ++qb) {
      const int qs0 = q0 + 32 * qb;
      if (qs0 >= q_hi || kw >= kv_end) continue;
      if constexpr (EXT > 0) {
        if (qs0 > wq_last || qs0 + 31 < wq_first) continue;  // no row of this step sees the wave's keys
      }
      if constexpr (EXT == 2) {
        // S = Q K^T and dP = dO V^T first, then one pass: modified score,
        // mask, P and dS = P (dP - delta) * scale * f'(s).
        f32x16 sx = f32x16{}, dpx = f32x16{};
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const typename E::v8 qf = E::as8(*(const u32x4*)(qs + qb * 32 * ROWB + off.row[kk]));
          sx = E::mma32(qf, kf[kk], sx);
        }
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const typename E::v8 df = E::as8(*(const u32x4*)(dos + qb * 32 * ROWB + off.row[kk]));
          dpx = E::mma32(df, vf[kk], dpx);
        }
        const HeadMods hm = head_mods(a.m, h);
        ext_scores_S<BIAS>(a, b, hm, key, qlo, qhi, segk, sx, qs0, half, bbase,
                           [&](int r, float x, float gg) {
                             const int ql = 32 * qb + 8 * (r >> 2) + 4 * half + (r & 3);
                             const float p = fast_exp2(fmaf(x, cx, -lsm[ql]));
                             sx[r] = p;
                             dpx[r] = p * fmaf(dpx[r], a.scale, -dlm[ql]) * gg;
                           });
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const typename E::v8 pf = pack_step<E>(sx, c);
          const typename E::v8 dsf = pack_step<E>(dpx, c);
#pragma unroll
          for (int db = 0; db < D / 32; ++db) {
            accv[db] = E::mma32(read_t<E, D>(dos, 32 * qb + 16 * c, off.tlo[db], off.thi[db]), pf, accv[db]);
            acck[db] = E::mma32(read_t<E, D>(qs, 32 * qb + 16 * c, off.tlo[db], off.thi[db]), dsf, acck[db]);
          }
        }
        continue;
      }
      if (EXT == 0 && a.causal && qs0 + 31 < kw) continue;  // every query before this wave's first key

      // S[query][key] = Q K^T: register r holds query qs0 + 8*(r/4) + 4*half + r%4
      // of key `key`.
      f32x16 s = f32x16{};
#pragma unroll
      for (int k = 0; k < D / 16; ++k) {
        const typename E::v8 qf = E::as8(*(const u32x4*)(qs + qb * 32 * ROWB + off.row[k]));
        s = E::mma32(qf, kf[k], s);
      }
      if constexpr (BIAS) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qr = qs0 + 8 * (r >> 2) + 4 * half + (r & 3);
          const float bv = (qr < a.Lq && key < a.Lk) ? bbase[(size_t)qr * a.Lk + key] : 0.f;
          s[r] = fmaf(s[r], a.scale, bv);
        }
      }
      if constexpr (EXT == 1)
        ext_mask_S(s, qs0, half, qlo, qhi, !(kw + 31 < kv_end && qs0 >= qlo_last && qs0 + 31 <= qhi_first));
      const bool need_mask = EXT == 0 && ((a.causal && qs0 < kw + 31) || (kw + 32 > kv_end) || (qs0 + 32 > q_hi));
      if (need_mask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qr = qs0 + 8 * (r >> 2) + 4 * half + (r & 3);
          const bool keep = key < kv_end && qr < q_hi && (!a.causal || qr >= key);
          if (!keep) s[r] = -INFINITY;
        }
      }
      // P, and dV^T[d][key] += dO^T P
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const f32x4 l4 = *(const f32x4*)(lsm + 32 * qb + 8 * gq + 4 * half);
#pragma unroll
        for (int j = 0; j < 4; ++j) s[4 * gq + j] = fast_exp2(fmaf(s[4 * gq + j], cx, -l4[j]));
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const typename E::v8 pf = pack_step<E>(s, c);
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
          accv[db] = E::mma32(read_t<E, D>(dos, 32 * qb + 16 * c, off.tlo[db], off.thi[db]), pf, accv[db]);
      }
      // dP = dO V^T; dS = P (dP - delta) * scale; dK^T[d][key] += Q^T dS
      f32x16 dp = f32x16{};
#pragma unroll
      for (int k = 0; k < D / 16; ++k) {
        const typename E::v8 df = E::as8(*(const u32x4*)(dos + qb * 32 * ROWB + off.row[k]));
        dp = E::mma32(df, vf[k], dp);
      }
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const f32x4 d4 = *(const f32x4*)(dlm + 32 * qb + 8 * gq + 4 * half);
#pragma unroll
        for (int j = 0; j < 4; ++j) s[4 * gq + j] = s[4 * gq + j] * fmaf(dp[4 * gq + j], a.scale, -d4[j]);
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const typename E::v8 dsf = pack_step<E>(s, c);
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
          acck[db] = E::mma32(read_t<E, D>(qs, 32 * qb + 16 * c, off.tlo[db], off.thi[db]), dsf, acck[db]);
      }
    }
  };

  // this group's steps NG*s + gi: n_loc of them; n_steps (the same for every
  // group) keeps the barriers in step
  const int n_loc = (n_tiles - gi + NG - 1) / NG;
  const int n_steps = (n_tiles + NG - 1) / NG;
  if (n_loc > 0) issue(gi, st0);
  for (int s = 0; s < n_steps; s += 2) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (s + 1 < n_loc) issue(NG * (s + 1) + gi, st1);
    if (s < n_loc) compute(NG * s + gi, smem0);
    if (s + 1 >= n_steps) break;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (s + 2 < n_loc) issue(NG * (s + 2) + gi, st0);
    if (s + 1 < n_loc) compute(NG * (s + 1) + gi, smem1);
  }
  if constexpr (NG > 1) {
    // Group 1 hands its dK^T / dV^T sums to group 0 through LDS, lane by lane
    // in the same register layout: 16-byte quads [D/32 * 4][4 waves][64 lanes],
    // dK over stage 0, dV over stage 1.
    static_assert((D / 32) * 4 * 256 * 16 <= NG * STAGE_B, "hand-off fits");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // every wave is done with the rings
    f32x4* xk = (f32x4*)smem0 + w * 64 + lane;
    f32x4* xv = (f32x4*)smem1 + w * 64 + lane;
    if (gi == 1) {
#pragma unroll
      for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int r = 0; r < 16; r += 4) {
          xk[(4 * i + r / 4) * 256] = f32x4{acck[i][r], acck[i][r + 1], acck[i][r + 2], acck[i][r + 3]};
          xv[(4 * i + r / 4) * 256] = f32x4{accv[i][r], accv[i][r + 1], accv[i][r + 2], accv[i][r + 3]};
        }
    }
    __syncthreads();
    if (gi == 1) return;
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        const f32x4 k1 = xk[(4 * i + r / 4) * 256], v1 = xv[(4 * i + r / 4) * 256];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acck[i][r + j] += k1[j];
          accv[i][r + j] += v1[j];
        }
      }
  }

  // dK, dV rows of this lane's key (zeros for keys past the valid length).
  if (key < a.Lk) {
    const size_t koff = ((size_t)(b * a.Lk + key) * a.Hkv + hkv) * D;
    uint16_t* dkrow = (uint16_t*)ba.dk + koff;
    uint16_t* dvrow = (uint16_t*)ba.dv + koff;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        u32x2 pk, pv;
        pk[0] = E::pack2(acck[db][4 * gq], acck[db][4 * gq + 1]);
        pk[1] = E::pack2(acck[db][4 * gq + 2], acck[db][4 * gq + 3]);
        pv[0] = E::pack2(accv[db][4 * gq], accv[db][4 * gq + 1]);
        pv[1] = E::pack2(accv[db][4 * gq + 2], accv[db][4 * gq + 3]);
        *(u32x2*)(dkrow + db * 32 + 8 * gq + 4 * half) = pk;
        *(u32x2*)(dvrow + db * 32 + 8 * gq + 4 * half) = pv;
      }
  }
}

// ---------------------------------------------------------------------------
// fp32 path: v_mfma_f32_32x32x2f32 (full fp32 products) for every product.
// One MFMA step contracts two indices, one per wave half.  Products whose
// contraction runs over the head dim take half rows (half 0: dims s, half 1:
// dims D/2 + s) as in the fp32 forward; products whose contraction runs over
// keys or queries take the pair (register r, half 0), (r, half 1) of a 32x32
// C block as the two indices, so their A operand is one float of a row-major
// tile.  Tiles are staged through registers into LDS rows padded to D + 4
// floats (16-byte reads of 16 consecutive rows hit distinct banks).
// ---------------------------------------------------------------------------
template <int D, int BIAS, int EXT>
__global__ __launch_bounds__(kThreads, 1) void flash_bwd_dq_f32_kernel(FlashBwdArgs ba) {
  constexpr bool HB = BIAS != 0, DB = BIAS == 2;  // as in flash_bwd_dq_kernel
  const FlashArgs& a = ba.f;
  constexpr int BK = (D == 128) ? 32 : 64;
  constexpr int KS = D + 4;
  constexpr int DC = D / 4;
  constexpr int PER_T = BK * DC / kThreads;
  static_assert(PER_T >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) float k_lds[2][BK * KS];
  __shared__ __attribute__((aligned(16))) float v_lds[2][BK * KS];

  BlockGeom g = block_geom(a);
  if constexpr (EXT > 0) ext_block_range(a, g, BK);
  const int tid = threadIdx.x, lane = tid & 63;
  const int col = lane & 31, half = lane >> 5;
  const size_t kv_row = (size_t)a.Hkv * D;
  const float* Kb = (const float*)a.k + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * D;
  const float* Vb = (const float*)a.v + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * D;
  const bool row_in = g.qi < a.Lq;
  const bool row_ok = g.qi < g.q_hi;

  float qf[D / 2], dof[D / 2];
  float dsum = 0.f;
  {
    const size_t roff = ((size_t)(g.b * a.Lq + (row_in ? g.qi : 0)) * a.Hq + g.h) * D + half * (D / 2);
    const float* qrow = (const float*)a.q + roff;
    const float* drow = (const float*)ba.dout + roff;
    const float* orow = (const float*)a.o + roff;
#pragma unroll
    for (int s = 0; s < D / 8; ++s) {
      f32x4 rq = {0.f, 0.f, 0.f, 0.f}, rd = rq, ro = rq;
      if (row_in) {
        rq = *(const f32x4*)(qrow + 4 * s);
        rd = *(const f32x4*)(drow + 4 * s);
        ro = *(const f32x4*)(orow + 4 * s);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        qf[4 * s + j] = rq[j];
        dof[4 * s + j] = rd[j];
        dsum = fmaf(ro[j], rd[j], dsum);
      }
    }
  }
  const float delta = xor32_sum(dsum);
  const float dsc = delta * a.scale;  // the workspace holds delta * sm_scale
  float lse2 = 0.f;
  const size_t lidx = ((size_t)g.b * a.Hq + g.h) * a.Lq + g.qi;
  if (row_in) {
    lse2 = a.lse[lidx] * kLog2e;
    if (half == 0) {
      ba.delta[lidx] = dsc;
      ba.lse2[lidx] = lse2;
    }
  }
  const float* brow = nullptr;
  if constexpr (HB) {
    brow = a.bias + (size_t)g.b * a.bias_bstride + (size_t)g.h * a.bias_hstride +
           (size_t)(row_in ? g.qi : 0) * a.Lk;
  }
  const bool bias_vec = (a.Lk & 3) == 0;
  const float cx = (HB || EXT == 2) ? kLog2e : a.scale * kLog2e;
  ExtRows er;
  if constexpr (EXT > 0) er = ext_rows(a, g);

  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16{};
  const int t_begin = g.kv_begin / BK;
  const int n_tiles = max((g.kv_stop + BK - 1) / BK - t_begin, 0);
  const int q_last_w = g.qw + 31;

  f32x4 kreg[PER_T], vreg[PER_T];
  auto load_tile = [&](int t) {
    const int k0 = (t_begin + t) * BK;
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int u = tid + kThreads * i;
      const int kk = k0 + u / DC, dc = u % DC;
      f32x4 rk = {0.f, 0.f, 0.f, 0.f}, rv = rk;
      if (kk < g.kv_stop) {
        rk = *(const f32x4*)(Kb + (size_t)kk * kv_row + dc * 4);
        rv = *(const f32x4*)(Vb + (size_t)kk * kv_row + dc * 4);
      }
      kreg[i] = rk;
      vreg[i] = rv;
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int u = tid + kThreads * i;
      *(f32x4*)(&k_lds[buf][(u / DC) * KS + (u % DC) * 4]) = kreg[i];
      *(f32x4*)(&v_lds[buf][(u / DC) * KS + (u % DC) * 4]) = vreg[i];
    }
  };

  auto compute = [&](int t, int buf) {
    const int k0 = (t_begin + t) * BK;
    if constexpr (EXT > 0) {
      if (!er.any || k0 > er.hi_last || k0 + BK - 1 < er.lo_first) return;
    } else {
      if (a.causal && k0 > q_last_w) return;
    }
    const float* kl = k_lds[buf];
    const float* vl = v_lds[buf];
    f32x16 s[BK / 32], dp[BK / 32];
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb) {
      s[kb] = f32x16{};
      dp[kb] = f32x16{};
      const float* kp = kl + (kb * 32 + col) * KS + half * (D / 2);
      const float* vp = vl + (kb * 32 + col) * KS + half * (D / 2);
#pragma unroll
      for (int st4 = 0; st4 < D / 8; ++st4) {
        const f32x4 kf = *(const f32x4*)(kp + 4 * st4);
        const f32x4 vf = *(const f32x4*)(vp + 4 * st4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s[kb] = mfma32x32x2f32(kf[j], qf[4 * st4 + j], s[kb]);
          dp[kb] = mfma32x32x2f32(vf[j], dof[4 * st4 + j], dp[kb]);
        }
      }
    }
    f32x16 dbv[DB ? BK / 32 : 1];
    if constexpr (EXT == 2) {
      ext_scores_sT<BK / 32, HB>(a, g, er, s, k0, half, brow, row_in,
                                 [&](int kb, int r, float x, float gg) {
                                   const float p = fast_exp2(fmaf(x, cx, -lse2));
                                   const float t = p * (dp[kb][r] - delta);
                                   if constexpr (DB) dbv[kb][r] = t;
                                   s[kb][r] = t * a.scale * gg;
                                 });
    } else {
    if constexpr (HB) {
#pragma unroll
      for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int kk = k0 + kb * 32 + 8 * gq + 4 * half;
          f32x4 bv = {0.f, 0.f, 0.f, 0.f};
          if (row_in) bv = bias_vec ? load_bias4<true>(brow, kk, a.Lk) : load_bias4<false>(brow, kk, a.Lk);
#pragma unroll
          for (int j = 0; j < 4; ++j) s[kb][4 * gq + j] = fmaf(s[kb][4 * gq + j], a.scale, bv[j]);
        }
    }
    if constexpr (EXT == 1) ext_mask_sT<BK / 32>(g, er, s, k0, half);
    const bool need_mask = EXT == 0 && ((k0 + BK > g.kv_end) || (a.causal && k0 + BK - 1 > g.qw) ||
                                        (g.qw + 31 >= g.q_hi));
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = k0 + kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          const bool keep = row_ok && kk < g.kv_end && (!a.causal || kk <= g.qi);
          if (!keep) s[kb][r] = -INFINITY;
        }
    }
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(s[kb][r], cx, -lse2));
        if constexpr (DB) {
          const float t = p * (dp[kb][r] - delta);
          dbv[kb][r] = t;
          s[kb][r] = t * a.scale;
        } else {
          s[kb][r] = p * fmaf(dp[kb][r], a.scale, -dsc);  // p (dp - delta) scale
        }
      }
    }
    if constexpr (DB) store_dbias<BK / 32>(ba, g, dbv, k0, half, row_in);
    // dQ^T[d][query] += K^T dS^T: step (kb, r) contracts keys (r, half 0/1).
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          acc[db] = mfma32x32x2f32(kl[key * KS + db * 32 + col], s[kb][r], acc[db]);
        }
  };

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    if (t + 1 < n_tiles) load_tile(t + 1);
    compute(t, t & 1);
    if (t + 1 < n_tiles) store_tile((t + 1) & 1);
    __syncthreads();
  }

  if (row_in) {
    float* drow = (float*)ba.dq + ((size_t)(g.b * a.Lq + g.qi) * a.Hq + g.h) * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = acc[db][4 * gq + j];
        *(f32x4*)(drow + db * 32 + 8 * gq + 4 * half) = v;
      }
  }
}

template <int D, bool BIAS, int EXT>
__global__ __launch_bounds__(kThreads, 1) void flash_bwd_dkdv_f32_kernel(FlashBwdArgs ba) {
  const FlashArgs& a = ba.f;
  constexpr int BQ = 32;  // queries per stage (one 32-query step)
  constexpr int KS = D + 4;
  constexpr int DC = D / 4;
  constexpr int PER_T = BQ * DC / kThreads;
  static_assert(PER_T >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) float q_lds[2][BQ * KS];
  __shared__ __attribute__((aligned(16))) float d_lds[2][BQ * KS];
  __shared__ __attribute__((aligned(16))) float ld_lds[2][2 * BQ];  // lse*log2e, delta * sm_scale

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int BH = a.B * a.Hkv;
  const int bh = blockIdx.x % BH;
  const int k0 = (blockIdx.x / BH) * kBKV;
  const int b = bh / a.Hkv, hkv = bh % a.Hkv;
  const int G = a.Hq / a.Hkv;
  const int kw = k0 + 32 * w;
  const int key = kw + col;
  int kv_end = min(a.Lk, a.kv_valid);
  if (a.kv_lengths) kv_end = min(kv_end, max(a.kv_lengths[b], 0));
  const int q_hi = min(a.Lq, a.q_valid);
  int q_begin = a.causal ? (k0 / BQ) * BQ : 0;
  int q_end = q_hi;
  int qlo = 0, qhi = q_hi - 1, wq_first = 0, wq_last = q_hi - 1, segk = 0;
  int qhi_first = q_hi - 1, qlo_last = 0;  // rows seen by every key of the wave: [qlo_last, qhi_first]
  if constexpr (EXT > 0) {
    q_end = q_begin = 0;
    if (k0 < kv_end) {
      int a0, a1, b0, b1;
      key_bounds(a.m, a.causal, b, kv_end, q_hi, k0, a0, a1);
      key_bounds(a.m, a.causal, b, kv_end, q_hi, min(k0 + kBKV, kv_end) - 1, b0, b1);
      q_begin = max(a0, 0);
      q_end = b1 + 1;
    }
    key_bounds(a.m, a.causal, b, kv_end, q_hi, key, qlo, qhi);
    if (kw < kv_end) {
      key_bounds(a.m, a.causal, b, kv_end, q_hi, kw, wq_first, qhi_first);
      key_bounds(a.m, a.causal, b, kv_end, q_hi, min(kw + 32, kv_end) - 1, qlo_last, wq_last);
    }
    if (a.m.seg_k && key < a.Lk) segk = a.m.seg_k[(size_t)b * a.Lk + key];
  }
  const int n_qt = (k0 < kv_end && q_end > q_begin) ? (q_end - q_begin + BQ - 1) / BQ : 0;
  const int n_tiles = G * n_qt;

  float kf[D / 2], vf[D / 2];
  {
    const bool kin = key < a.Lk;
    const size_t koff = ((size_t)(b * a.Lk + (kin ? key : 0)) * a.Hkv + hkv) * D + half * (D / 2);
    const float* krow = (const float*)a.k + koff;
    const float* vrow = (const float*)a.v + koff;
#pragma unroll
    for (int s = 0; s < D / 8; ++s) {
      f32x4 rk = {0.f, 0.f, 0.f, 0.f}, rv = rk;
      if (kin) {
        rk = *(const f32x4*)(krow + 4 * s);
        rv = *(const f32x4*)(vrow + 4 * s);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kf[4 * s + j] = rk[j];
        vf[4 * s + j] = rv[j];
      }
    }
  }
  const float cx = (BIAS || EXT == 2) ? kLog2e : a.scale * kLog2e;
  const size_t q_row = (size_t)a.Hq * D;

  f32x16 acck[D / 32], accv[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    acck[i] = f32x16{};
    accv[i] = f32x16{};
  }

  f32x4 qreg[PER_T], dreg[PER_T];
  float lreg = 0.f;
  // last query tile first, heads innermost (as the bf16 kernel)
  auto tile_head = [&](int t) { return hkv * G + t % G; };
  auto tile_q0 = [&](int t) { return q_begin + (n_qt - 1 - t / G) * BQ; };
  auto load_tile = [&](int t) {
    const int h = tile_head(t), q0 = tile_q0(t);
    const float* Qb = (const float*)a.q + ((size_t)b * a.Lq * a.Hq + h) * D;
    const float* Db = (const float*)ba.dout + ((size_t)b * a.Lq * a.Hq + h) * D;
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int u = tid + kThreads * i;
      const int qq = q0 + u / DC, dc = u % DC;
      f32x4 rq = {0.f, 0.f, 0.f, 0.f}, rd = rq;
      if (qq < a.Lq) {
        rq = *(const f32x4*)(Qb + (size_t)qq * q_row + dc * 4);
        rd = *(const f32x4*)(Db + (size_t)qq * q_row + dc * 4);
      }
      qreg[i] = rq;
      dreg[i] = rd;
    }
    lreg = 0.f;
    if (tid < 2 * BQ) {
      const int qq = q0 + (tid % BQ);
      const size_t li = ((size_t)b * a.Hq + h) * a.Lq + qq;
      if (qq < a.Lq) lreg = tid < BQ ? ba.lse2[li] : ba.delta[li];
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int u = tid + kThreads * i;
      *(f32x4*)(&q_lds[buf][(u / DC) * KS + (u % DC) * 4]) = qreg[i];
      *(f32x4*)(&d_lds[buf][(u / DC) * KS + (u % DC) * 4]) = dreg[i];
    }
    if (tid < 2 * BQ) ld_lds[buf][tid] = lreg;
  };

  auto compute = [&](int t, int buf) {
    const int h = tile_head(t), q0 = tile_q0(t);
    if (q0 >= q_hi || kw >= kv_end) return;
    if constexpr (EXT > 0) {
      if (q0 > wq_last || q0 + BQ - 1 < wq_first) return;  // no row of this step sees the wave's keys
    } else {
      if (a.causal && q0 + BQ - 1 < kw) return;  // every query before this wave's first key
    }
    const float* ql = q_lds[buf];
    const float* dl = d_lds[buf];
    const float* lsm = ld_lds[buf];
    // S[query][key] = Q K^T and dP = dO V^T; register r holds query
    // q0 + 8*(r/4) + 4*half + r%4 of key `key`.
    f32x16 s = f32x16{}, dp = f32x16{};
    {
      const float* qp = ql + col * KS + half * (D / 2);
      const float* dpp = dl + col * KS + half * (D / 2);
#pragma unroll
      for (int st4 = 0; st4 < D / 8; ++st4) {
        const f32x4 qv = *(const f32x4*)(qp + 4 * st4);
        const f32x4 dv4 = *(const f32x4*)(dpp + 4 * st4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s = mfma32x32x2f32(qv[j], kf[4 * st4 + j], s);
          dp = mfma32x32x2f32(dv4[j], vf[4 * st4 + j], dp);
        }
      }
    }
    f32x16 ds;
    if constexpr (EXT == 2) {
      const float* bbase = nullptr;
      if constexpr (BIAS) bbase = a.bias + (size_t)b * a.bias_bstride + (size_t)h * a.bias_hstride;
      const HeadMods hm = head_mods(a.m, h);
      ext_scores_S<BIAS>(a, b, hm, key, qlo, qhi, segk, s, q0, half, bbase,
                         [&](int r, float x, float gg) {
                           const int qi = 8 * (r >> 2) + 4 * half + (r & 3);
                           const float p = fast_exp2(fmaf(x, cx, -lsm[qi]));
                           s[r] = p;
                           ds[r] = p * fmaf(dp[r], a.scale, -lsm[BQ + qi]) * gg;
                         });
    } else {
    if constexpr (BIAS) {
      const float* bbase = a.bias + (size_t)b * a.bias_bstride + (size_t)h * a.bias_hstride;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qr = q0 + 8 * (r >> 2) + 4 * half + (r & 3);
        const float bv = (qr < a.Lq && key < a.Lk) ? bbase[(size_t)qr * a.Lk + key] : 0.f;
        s[r] = fmaf(s[r], a.scale, bv);
      }
    }
    if constexpr (EXT == 1)
      ext_mask_S(s, q0, half, qlo, qhi, !(kw + 31 < kv_end && q0 >= qlo_last && q0 + BQ - 1 <= qhi_first));
    const bool need_mask = EXT == 0 && ((a.causal && q0 < kw + 31) || (kw + 32 > kv_end) || (q0 + BQ > q_hi));
    if (need_mask) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qr = q0 + 8 * (r >> 2) + 4 * half + (r & 3);
        const bool keep = key < kv_end && qr < q_hi && (!a.causal || qr >= key);
        if (!keep) s[r] = -INFINITY;
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qi = 8 * (r >> 2) + 4 * half + (r & 3);
      const float p = fast_exp2(fmaf(s[r], cx, -lsm[qi]));
      s[r] = p;
      ds[r] = p * fmaf(dp[r], a.scale, -lsm[BQ + qi]);
    }
    }
    // dV^T[d][key] += dO^T P and dK^T[d][key] += Q^T dS: step r contracts
    // queries (r, half 0/1).
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qi = 8 * (r >> 2) + 4 * half + (r & 3);
        accv[db] = mfma32x32x2f32(dl[qi * KS + db * 32 + col], s[r], accv[db]);
        acck[db] = mfma32x32x2f32(ql[qi * KS + db * 32 + col], ds[r], acck[db]);
      }
  };

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    if (t + 1 < n_tiles) load_tile(t + 1);
    compute(t, t & 1);
    if (t + 1 < n_tiles) store_tile((t + 1) & 1);
    __syncthreads();
  }

  if (key < a.Lk) {
    const size_t koff = ((size_t)(b * a.Lk + key) * a.Hkv + hkv) * D;
    float* dkrow = (float*)ba.dk + koff;
    float* dvrow = (float*)ba.dv + koff;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        f32x4 vk, vv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          vk[j] = acck[db][4 * gq + j];
          vv[j] = accv[db][4 * gq + j];
        }
        *(f32x4*)(dkrow + db * 32 + 8 * gq + 4 * half) = vk;
        *(f32x4*)(dvrow + db * 32 + 8 * gq + 4 * half) = vv;
      }
  }
}

template <auto K>
static int launch_dq(const FlashBwdArgs& a, hipStream_t stream, int threads = kThreads) {
  const long blocks = (long)a.f.n_qtiles * a.f.B * a.f.Hq;
  launch_kernel<K>(dim3((unsigned)blocks), dim3(threads), 0, stream, a);
  return check_launch("pjx_flash_bwd (dq)");
}

template <auto K>
static int launch_dkdv(const FlashBwdArgs& a, hipStream_t stream, int threads = kThreads) {
  const long blocks = (long)((a.f.Lk + kBKV - 1) / kBKV) * a.f.B * a.f.Hkv;
  launch_kernel<K>(dim3((unsigned)blocks), dim3(threads), 0, stream, a);
  return check_launch("pjx_flash_bwd (dk, dv)");
}

// dK/dV at D = 256 without extended masks (16-bit): flash_bwd_dkdv_kernel at
// one wave per SIMD, in flash_bwd256.hip (built in the default MFMA register
// form, which this kernel needs; the rest of the backward is built in the
// VGPR form).  Returns a PJX_* status.
int launch_dkdv256(const FlashBwdArgs& a, bool f16, bool hb, hipStream_t s);

// fp32 backward at head dim 256 (dQ then dK/dV, flash_f32_wide.hip).
int run_flash_f32_wide_bwd(const FlashBwdArgs& ba, hipStream_t s);

}  // namespace pjx
