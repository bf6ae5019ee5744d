// Flash-attention forward for gfx950 (MI355X): causal / KV-length / static
// length masks and an fp32 dense additive bias, bf16 or fp32 inputs.
//
// Semantics follow probjax's XLA attention reference
// (probjax/nn/pallas_kernels/kernels/attention_xla.py:339-429): scores are
// sm_scale * q.k in fp32, then the bias, then the mask (masked -> -inf); an
// online softmax in the exp2 domain (as the Pallas kernel,
// kernels/attention.py:483-494); P is rounded to bf16 before the P.V product
// in bf16 mode (attention_xla.py:349; attention.py:506); rows with no valid
// key give 0 (attention_xla.py:417-420).
//
// Work decomposition: one workgroup = 4 waves = 128 query rows of one
// (batch, head); each wave owns 32 rows.  Per KV tile of BK keys a wave
// computes S^T = K Q^T with the keys as MFMA rows, so every lane holds the
// scores of ONE query for 16 keys per 32-key block: the row max / row sum are
// lane-local plus one v_permlane32_swap, with no shuffle trees.  P feeds
// O^T = V^T P^T straight from registers (the lane layout of S^T's C operand is
// the B-operand layout of the next MFMA up to a key permutation that V^T's
// A operand reproduces), so the per-row rescale and 1/l are lane-local too.
// bf16: K and V tiles go HBM -> LDS by buffer loads that write LDS directly,
// both stored row-major; the A operand of P.V (V^T) comes from transposing
// LDS reads of the row-major V tile.  fp32: tiles are staged through
// registers.  Either way LDS holds two tiles, the loads of tile t+1 are in
// flight while tile t is computed, and there is one barrier per tile.
//
// This file also holds the fp32 kernel for small grids (each query block's
// keys split over the waves of a workgroup) and pjx_flash_fwd, which picks
// the kernel; the bf16 dense-bias kernel is in flash_bias_ring.hip.
//
// Grid: one workgroup per (q tile, batch, head), ordered heaviest causal
// q-tile first (longest-processing-time order), and batch*head fastest so
// that every q-tile of one (batch, head) lands on the same XCD (workgroups are
// dispatched round-robin over the 8 XCDs; batch*head is a multiple of 8 in
// the configs) and shares its K/V in that XCD's L2.
#include "flash_common.h"

namespace pjx {

// ---------------------------------------------------------------------------
// bf16 path: v_mfma_f32_32x32x16_bf16 for both products.
//
// K/V tiles of BK keys go HBM -> LDS with buffer loads that write LDS
// directly (no VGPR staging), two stages: the loads of tile t+1 are issued
// right after the barrier that opens tile t, so they overlap its arithmetic.
// Each buffer resource spans only the tile's valid rows, so rows past the
// last visited key read as zero without any predication.  Per-lane LDS
// offsets are computed once; the key loop does no address arithmetic.
//
// LDS layout: row-major [key][dim] rows of D*2 bytes, 16-byte chunks XOR-
// swizzled per row (K: chunk ^ (row & (NC-1)); V: chunk ^ f(row) chosen so a
// transposing read of 4 rows x 32 bytes per 16 lanes hits distinct banks).
// K fragments are ds_read_b128; V^T fragments come from ds_read_b64_tr_b16
// straight out of the row-major V tile.
//
// Softmax: the running max used for exponentiation is only raised when a
// row's tile max exceeds it by more than kRescaleLog2 (wave-uniform branch),
// so the O rescale (D/2 multiplies per lane) runs on a few tiles per row
// instead of every tile; P stays <= 2^kRescaleLog2, exact in bf16 range.  The
// normalised output is the same softmax: O / l with l accumulated against the
// same reference max.
// ---------------------------------------------------------------------------


template <typename E, int D, bool BIAS, int EXT>
__global__ __launch_bounds__(kThreads, 2) void flash_fwd_bf16_kernel(FlashArgs a) {
  using T = Bf16Tile<D>;
  constexpr int BK = T::BK, ROWB = T::ROWB, TILE_B = T::TILE_B, STAGE_B = T::STAGE_B;
  // Two stages as distinct LDS objects: the compiler can then prove that the
  // buffer->LDS loads in flight for one stage do not alias reads of the other
  // (one array indexed by stage would make it wait for those loads first).
  __shared__ __attribute__((aligned(1024))) unsigned char smem0[STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char smem1[STAGE_B];

  BlockGeom g = block_geom(a);
  if constexpr (EXT > 0) ext_block_range(a, g, BK);
  const int tid = threadIdx.x, lane = tid & 63;
  // Wave index and the wave's first row as wave-uniform (scalar) values, so
  // that branches on them are scalar branches.
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  g.qw = __builtin_amdgcn_readfirstlane(g.qw);
  const int col = lane & 31, half = lane >> 5;
  const uint32_t rowstride = (uint32_t)a.Hkv * D * 2;
  const unsigned char* Kb = (const unsigned char*)a.k + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * ROWB;
  const unsigned char* Vb = (const unsigned char*)a.v + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * ROWB;
  const bool row_in = g.qi < a.Lq;
  const bool row_ok = g.qi < g.q_hi;

  // Q^T as the B operand: lane holds query `col`, dims 16*s + 8*half + [0,8).
  typename E::v8 qf[D / 16];
  {
    const uint16_t* qrow =
        (const uint16_t*)a.q + ((size_t)(g.b * a.Lq + (row_in ? g.qi : 0)) * a.Hq + g.h) * D;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row_in) raw = *(const u32x4*)(qrow + 16 * s + 8 * half);
      qf[s] = E::as8(raw);
    }
  }
  const float* brow = nullptr;
  if constexpr (BIAS) {
    brow = a.bias + (size_t)g.b * a.bias_bstride + (size_t)g.h * a.bias_hstride +
           (size_t)(row_in ? g.qi : 0) * a.Lk;
  }
  const bool bias_vec = (a.Lk & 3) == 0;
  // score units -> log2 units (the scale is applied to the score itself when
  // a bias or modifier is added to it)
  const float cx = (BIAS || EXT == 2) ? kLog2e : a.scale * kLog2e;
  ExtRows er;
  if constexpr (EXT > 0) er = ext_rows(a, g);

  // Per-lane byte offsets, fixed for the whole key loop.
  uint32_t voffK[T::NLD], voffV[T::NLD];
#pragma unroll
  for (int j = 0; j < T::NLD; ++j) {
    const int r = 16 * w + T::RPI * j + lane / T::NC, slot = lane % T::NC;
    voffK[j] = r * rowstride + 16 * (slot ^ T::swz_k(r));
    voffV[j] = r * rowstride + 16 * (slot ^ T::swz_v(r));
  }
  uint32_t offK[D / 16];  // K row `col` (of a 32-key block), dims 16*st + 8*half
#pragma unroll
  for (int st = 0; st < D / 16; ++st) offK[st] = col * ROWB + 16 * ((2 * st + half) ^ T::swz_k(col));
  uint32_t offV[D / 32];  // transposing-read source of this lane for output dims 32*db..
  {
    const int s16 = lane & 15, grp = lane >> 4;
    const int r = 4 * half + s16 / 4;  // row within a 16-key step (mod 4 = s16/4)
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int chunk = 4 * db + 2 * (grp & 1) + ((s16 & 3) >> 1);
      offV[db] = r * ROWB + 16 * (chunk ^ T::swz_v(r)) + 8 * (s16 & 1);
    }
  }

  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16{};
  float m_run = kMaxInit, l_run = 0.f;

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
      buffer_load_lds16(rk, ks + r0 * ROWB, voffK[j]);
      buffer_load_lds16(rv, ks + TILE_B + r0 * ROWB, voffV[j]);
    }
  };

  auto compute = [&](int t, const unsigned char* ks) {
    const int k0 = (t_begin + t) * BK;
    if constexpr (EXT > 0) {
      // tile outside every row of this wave
      if (!er.any || k0 > er.hi_last || k0 + BK - 1 < er.lo_first) return;
    } else {
      if (a.causal && k0 > q_last_w) return;  // tile above this wave's diagonal
    }
    const unsigned char* vs = ks + TILE_B;

    // S^T[key][query] = K Q^T
    f32x16 s[BK / 32];
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb) {
      s[kb] = f32x16{};
#pragma unroll
      for (int st = 0; st < D / 16; ++st) {
        const typename E::v8 kf = E::as8(*(const u32x4*)(ks + kb * 32 * ROWB + offK[st]));
        s[kb] = E::mma32(kf, qf[st], s[kb]);
      }
    }

    // Register r of block kb holds key k0 + kb*32 + 8*(r/4) + 4*half + r%4.
    if constexpr (EXT == 2) {
      ext_scores_sT<BK / 32, BIAS>(a, g, er, s, k0, half, brow, row_in,
                                   [&](int kb, int r, float x, float) { s[kb][r] = x; });
    } else if constexpr (BIAS) {
#pragma unroll
      for (int kb = 0; kb < BK / 32; ++kb) {
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int kk = k0 + kb * 32 + 8 * gq + 4 * half;
          f32x4 bv = {0.f, 0.f, 0.f, 0.f};
          if (row_in) bv = bias_vec ? load_bias4<true>(brow, kk, a.Lk) : load_bias4<false>(brow, kk, a.Lk);
#pragma unroll
          for (int j = 0; j < 4; ++j) s[kb][4 * gq + j] = fmaf(s[kb][4 * gq + j], a.scale, bv[j]);
        }
      }
    }
    if constexpr (EXT == 1) ext_mask_sT<BK / 32>(g, er, s, k0, half);
    const bool need_mask = EXT == 0 && ((k0 + BK > g.kv_end) || (a.causal && k0 + BK - 1 > g.qw) ||
                                        (g.qw + 31 >= g.q_hi));
    if (need_mask) {
      // Key k0 + 4*half + o (o = kb*32 + 8*(r/4) + r%4) is kept iff o <= lim.
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

    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
      for (int r = 0; r < 16; r += 2) mx = fmaxf(mx, fmaxf(s[kb][r], s[kb][r + 1]));
    const float mc = xor32_max(mx) * cx;
    if (wave_any(mc > m_run + kRescaleLog2)) {
      const float m_new = fmaxf(m_run, mc);
      const float corr = fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= corr;
#pragma unroll
      for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] *= corr;
    }
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(s[kb][r], cx, -m_run));
        rs += p;
        s[kb][r] = p;
      }
    l_run += rs;

    // P^T as the B operand, 16 keys per MFMA step c:
    // slot j <-> key 16c + 8*(j/4) + 4*half + j%4 (registers 8*(c%2)+j of block c/2).
    typename E::v8 pf[BK / 16];
#pragma unroll
    for (int c = 0; c < BK / 16; ++c) {
      u32x4 pk;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        pk[j] = E::pack2(s[c >> 1][8 * (c & 1) + 2 * j], s[c >> 1][8 * (c & 1) + 2 * j + 1]);
      pf[c] = E::as8(pk);
    }
    // O^T[d][query] += V^T P^T; A operand = V^T rows 32*db.., keys in P's slot order,
    // from two transposing reads (keys 16c + 4*half + [0,4) and 16c + 8 + 4*half + [0,4)).
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
#pragma unroll
      for (int c = 0; c < BK / 16; ++c) {
        const u32x2 lo = lds_read_tr16(vs + 16 * c * ROWB + offV[db]);
        const u32x2 hi = lds_read_tr16(vs + (16 * c + 8) * ROWB + offV[db]);
        const u32x4 av = {lo[0], lo[1], hi[0], hi[1]};
        acc[db] = E::mma32(E::as8(av), pf[c], acc[db]);
      }
    }
  };

  // Tile t lives in stage t % 2.  At the top of each step: this wave's loads of
  // tile t have landed (waitcnt), then every wave's have and every wave is done
  // reading the other stage (barrier), so tile t+1's loads can go there while
  // tile t is computed.
  if (n_tiles > 0) issue(0, smem0);
  for (int t = 0; t < n_tiles; t += 2) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t + 1 < n_tiles) issue(t + 1, smem1);
    compute(t, smem0);
    if (t + 1 >= n_tiles) break;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t + 2 < n_tiles) issue(t + 2, smem0);
    compute(t + 1, smem1);
  }

  const float l_tot = xor32_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row_in) {
    uint16_t* orow = (uint16_t*)a.o + ((size_t)(g.b * a.Lq + g.qi) * a.Hq + g.h) * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        u32x2 pk;
        pk[0] = E::pack2(acc[db][4 * gq] * inv, acc[db][4 * gq + 1] * inv);
        pk[1] = E::pack2(acc[db][4 * gq + 2] * inv, acc[db][4 * gq + 3] * inv);
        *(u32x2*)(orow + db * 32 + 8 * gq + 4 * half) = pk;
      }
    if (a.lse && half == 0)
      a.lse[((size_t)g.b * a.Hq + g.h) * a.Lq + g.qi] =
          l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : INFINITY;
  }
}

// ---------------------------------------------------------------------------
// bf16 without bias or extended masks (the headline case): the same
// decomposition with the key loop software-pipelined inside each wave.
// Iteration t issues S_{t+1} = K_{t+1} Q^T on the MFMA pipe in the same
// basic block as tile t's exponentials, row sums and packing, so a wave's own
// VALU work runs while its MFMAs execute; then O += P_t V_t.
//
// The 2-stage ring keeps K one tile ahead of V: after the barrier that opens
// iteration t, K_{t+2} goes into the K slot of stage t%2 (K_t was consumed by
// iteration t-1, which formed S_t) and V_{t+1} into the V slot of stage
// (t+1)%2 (V_{t-1} was consumed by iteration t-1).  Iteration t reads K_{t+1}
// and V_t, both loaded during iteration t-1.  S_{t+1} is formed even where
// this wave will not use it (past its causal diagonal, past the last tile):
// it reads whatever the slot holds and is discarded, so the block stays
// branch-free.
//
// G = 2 (small grids): 8 waves, two groups of 4 over the same 128 rows, group
// j taking the key tiles t with t % 2 == j through a ring of its own (the
// loop above in the group's local tile index, the barriers in step), then
// group 1 hands (max, sum, O) to group 0 through LDS.
// ---------------------------------------------------------------------------
template <typename E, int D, int BKT, int WPC, int G = 1>
__global__ __launch_bounds__(G * kThreads, WPC) void flash_fwd_bf16_pipe_kernel(FlashArgs a) {
  using T = Bf16Tile<D, BKT>;
  constexpr int RPW = BKT / 4;  // tile rows each wave loads
  static_assert(BKT % 32 == 0 && RPW % T::RPI == 0 && T::NLD >= 1, "tile rows per wave");
  static_assert(G == 1 || G == 2, "one or two groups");
  constexpr int BK = T::BK, ROWB = T::ROWB, TILE_B = T::TILE_B, STAGE_B = T::STAGE_B;
  __shared__ __attribute__((aligned(1024))) unsigned char smem0[G * STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char smem1[G * STAGE_B];

  BlockGeom g = block_geom(a);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w8 = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gi = G > 1 ? w8 >> 2 : 0;     // group: the key tiles t with t % G == gi
  const int w = G > 1 ? (w8 & 3) : w8;    // wave within the group: rows 32w .. of the q tile
  if constexpr (G > 1) {
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

  typename E::v8 qf[D / 16];
  {
    const uint16_t* qrow =
        (const uint16_t*)a.q + ((size_t)(g.b * a.Lq + (row_in ? g.qi : 0)) * a.Hq + g.h) * D;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row_in) raw = *(const u32x4*)(qrow + 16 * s + 8 * half);
      qf[s] = E::as8(raw);
    }
  }
  const float cx = a.scale * kLog2e;

  uint32_t voffK[T::NLD], voffV[T::NLD];
#pragma unroll
  for (int j = 0; j < T::NLD; ++j) {
    const int r = RPW * w + T::RPI * j + lane / T::NC, slot = lane % T::NC;
    voffK[j] = r * rowstride + 16 * (slot ^ T::swz_k(r));
    voffV[j] = r * rowstride + 16 * (slot ^ T::swz_v(r));
  }
  uint32_t offK[D / 16];
#pragma unroll
  for (int st = 0; st < D / 16; ++st) offK[st] = col * ROWB + 16 * ((2 * st + half) ^ T::swz_k(col));
  uint32_t offV[D / 32];
  {
    const int s16 = lane & 15, grp = lane >> 4;
    const int r = 4 * half + s16 / 4;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int chunk = 4 * db + 2 * (grp & 1) + ((s16 & 3) >> 1);
      offV[db] = r * ROWB + 16 * (chunk ^ T::swz_v(r)) + 8 * (s16 & 1);
    }
  }

  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16{};
  float m_run = kMaxInit, l_run = 0.f;
  float thr = -INFINITY;  // rescale when a raw row max exceeds (m_run + kRescaleLog2) / cx

  const int n_tiles = max((g.kv_stop + BK - 1) / BK, 0);
  const int q_last_w = g.qw + 31;
  // tiles this wave uses: a causal wave stops at the tile holding its last row
  const int n_w = a.causal ? min(n_tiles, q_last_w / BK + 1) : n_tiles;
  // this group's tiles G*s + gi: n_loc of them, the first n_wl used by this
  // wave; n_steps (the same for every group) keeps the barriers in step
  const int n_loc = (n_tiles - gi + G - 1) / G;
  const int n_wl = n_w > gi ? (n_w - gi + G - 1) / G : 0;
  const int n_steps = (n_tiles + G - 1) / G;

  auto issue = [&](const unsigned char* base, int t, unsigned char* dst, const uint32_t* voff) {
    const int k0 = t * BK;
    const int nvalid = min(BK, g.kv_stop - k0);
    const uint32_t bytes = (uint32_t)(nvalid - 1) * rowstride + ROWB;
    const rsrc_t rs = make_rsrc(base + (size_t)k0 * rowstride, bytes);
#pragma unroll
    for (int j = 0; j < T::NLD; ++j) buffer_load_lds16(rs, dst + (RPW * w + T::RPI * j) * ROWB, voff[j]);
  };

  auto qk = [&](const unsigned char* ks, f32x16* s) {
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb) {
      s[kb] = f32x16{};
#pragma unroll
      for (int st = 0; st < D / 16; ++st) {
        const typename E::v8 kf = E::as8(*(const u32x4*)(ks + kb * 32 * ROWB + offK[st]));
        s[kb] = E::mma32(kf, qf[st], s[kb]);
      }
    }
  };

  // Tile t's softmax and P.V, with S_{t+1} formed from ks_next alongside.
  auto step = [&](int t, f32x16* s, const unsigned char* vs, const unsigned char* ks_next, f32x16* sn) {
    const int k0 = t * BK;
    const bool need_mask = (k0 + BK > g.kv_end) || (a.causal && k0 + BK - 1 > g.qw) || (g.qw + 31 >= g.q_hi);
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
    // Row max as a chain of 3-input maxima, compared in raw score units with
    // the rescale threshold (m_run + kRescaleLog2) / cx kept from the last
    // rescale: no per-tile multiply.
    float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
      for (int r = (kb == 0 ? 2 : 0); r < 16; r += 2) mx = fmaxf(fmaxf(mx, s[kb][r]), s[kb][r + 1]);
    mx = xor32_max(mx);
    if (wave_any(mx > thr)) {
      const float m_new = fmaxf(m_run, mx * cx);
      const float corr = fast_exp2(m_run - m_new);
      m_run = m_new;
      thr = (m_run + kRescaleLog2) / cx;
      l_run *= corr;
#pragma unroll
      for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] *= corr;
    }
    // one basic block from here: S_{t+1} on the MFMA pipe under the exponentials
    qk(ks_next, sn);
    // two independent partial sums (the adds need not wait on each other)
    float rs0 = 0.f, rs1 = 0.f;
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = fast_exp2(fmaf(s[kb][r], cx, -m_run));
        const float p1 = fast_exp2(fmaf(s[kb][r + 1], cx, -m_run));
        rs0 += p0;
        rs1 += p1;
        s[kb][r] = p0;
        s[kb][r + 1] = p1;
      }
    l_run += rs0 + rs1;
    typename E::v8 pf[BK / 16];
#pragma unroll
    for (int c = 0; c < BK / 16; ++c) {
      u32x4 pk;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        pk[j] = E::pack2(s[c >> 1][8 * (c & 1) + 2 * j], s[c >> 1][8 * (c & 1) + 2 * j + 1]);
      pf[c] = E::as8(pk);
    }
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
#pragma unroll
      for (int c = 0; c < BK / 16; ++c) {
        const u32x2 lo = lds_read_tr16(vs + 16 * c * ROWB + offV[db]);
        const u32x2 hi = lds_read_tr16(vs + (16 * c + 8) * ROWB + offV[db]);
        const u32x4 av = {lo[0], lo[1], hi[0], hi[1]};
        acc[db] = E::mma32(E::as8(av), pf[c], acc[db]);
      }
    }
    // 32-key tiles: issue order of the block is each S_{t+1} MFMA followed by
    // 5 VALU instructions (tile t's scaling, exponentials, sums and packing),
    // then the P.V MFMAs each followed by one.  Left to itself the scheduler
    // places every exponential ahead of the MFMAs: measured 1.3-1.9% slower on
    // C2; the 64-key form is 5% faster left alone.
    if constexpr (BK == 32) {
      constexpr int NQK = D / 16, NPV = D / 16;
#pragma unroll
      for (int i = 0; i < NQK; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x402, 5, 0);  // VALU incl. transcendental
      }
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x402, 1, 0);
      }
    }
  };

  f32x16 sa[BK / 32], sb[BK / 32];
  if (n_tiles > 0) {
    if (n_loc > 0) {
      issue(Kb, gi, st0, voffK);
      issue(Vb, gi, st0 + TILE_B, voffV);
      if (n_loc > 1) issue(Kb, G + gi, st1, voffK);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (n_loc > 0) qk(st0, sa);
  }
  // Local tile s (global tile G*s + gi): K in stage s%2 until iteration s-1,
  // V in stage s%2 from iteration s.
  for (int s = 0; s < n_steps; s += 2) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (s + 2 < n_loc) issue(Kb, G * (s + 2) + gi, st0, voffK);
    if (s + 1 < n_loc) issue(Vb, G * (s + 1) + gi, st1 + TILE_B, voffV);
    if (s < n_wl) step(G * s + gi, sa, st0 + TILE_B, st1, sb);
    if (s + 1 >= n_steps) break;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (s + 3 < n_loc) issue(Kb, G * (s + 3) + gi, st1, voffK);
    if (s + 2 < n_loc) issue(Vb, G * (s + 2) + gi, st0 + TILE_B, voffV);
    if (s + 1 < n_wl) step(G * (s + 1) + gi, sb, st1 + TILE_B, st0, sa);
  }
  if constexpr (G > 1) {
    // Group 1 hands (max, sum, O) to group 0 through LDS, lane by lane in the
    // same register layout: O as 16-byte quads [D/32 * 4][4 waves][64 lanes]
    // over stage 0 (consecutive lanes, consecutive banks), (max, sum) in
    // stage 1; group 0 merges them.
    static_assert((D / 32) * 4 * 256 * 16 <= G * STAGE_B && 256 * 8 <= G * STAGE_B, "hand-off fits");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // every wave is done with the ring
    f32x4* xo = (f32x4*)smem0 + w * 64 + lane;
    float* xml = (float*)smem1 + 2 * (w * 64 + lane);
    if (gi == 1) {
#pragma unroll
      for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int r = 0; r < 16; r += 4)
          xo[(4 * i + r / 4) * 256] = f32x4{acc[i][r], acc[i][r + 1], acc[i][r + 2], acc[i][r + 3]};
      xml[0] = m_run;
      xml[1] = l_run;
    }
    __syncthreads();
    if (gi == 1) return;
    const float m1 = xml[0], l1 = xml[1];
    const float M = fmaxf(m_run, m1);
    const float f0 = fast_exp2(m_run - M), f1 = fast_exp2(m1 - M);
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        const f32x4 o1 = xo[(4 * i + r / 4) * 256];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][r + j] = fmaf(acc[i][r + j], f0, o1[j] * f1);
      }
    l_run = fmaf(l_run, f0, l1 * f1);
    m_run = M;
  }

  const float l_tot = xor32_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row_in) {
    uint16_t* orow = (uint16_t*)a.o + ((size_t)(g.b * a.Lq + g.qi) * a.Hq + g.h) * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        u32x2 pk;
        pk[0] = E::pack2(acc[db][4 * gq] * inv, acc[db][4 * gq + 1] * inv);
        pk[1] = E::pack2(acc[db][4 * gq + 2] * inv, acc[db][4 * gq + 3] * inv);
        *(u32x2*)(orow + db * 32 + 8 * gq + 4 * half) = pk;
      }
    if (a.lse && half == 0)
      a.lse[((size_t)g.b * a.Hq + g.h) * a.Lq + g.qi] =
          l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : INFINITY;
  }
}

// ---------------------------------------------------------------------------
// fp32 path: v_mfma_f32_32x32x2f32 (full fp32 products) for both products.
// The k index of one MFMA step is the wave half: half 0 contracts dim s,
// half 1 dim D/2 + s, so each lane reads a contiguous half row of K.  For
// P.V the step pairs key (r, half 0) with key (r, half 1) of the S^T layout,
// so V is read in its natural [key][dim] layout: no transpose needed.
// ---------------------------------------------------------------------------
template <int D, bool BIAS, int EXT>
__global__ __launch_bounds__(kThreads, 1) void flash_fwd_f32_kernel(FlashArgs a) {
  constexpr int BK = (D == 128) ? 32 : 64;
  constexpr int KS = D + 4;  // floats; b128 reads of 16 rows hit distinct banks
  constexpr int VS = D + 8;  // floats; rows 4 apart land 32 banks apart
  constexpr int DC = D / 4;  // float4 chunks per row
  constexpr int PER_T = BK * DC / kThreads;
  static_assert(PER_T >= 1, "tile shape");

  __shared__ __attribute__((aligned(16))) float k_lds[2][BK * KS];
  __shared__ __attribute__((aligned(16))) float v_lds[2][BK * VS];

  BlockGeom g = block_geom(a);
  if constexpr (EXT > 0) ext_block_range(a, g, BK);
  const int tid = threadIdx.x, lane = tid & 63;
  const int col = lane & 31, half = lane >> 5;
  const size_t kv_row = (size_t)a.Hkv * D;
  const float* Kb = (const float*)a.k + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * D;
  const float* Vb = (const float*)a.v + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * D;
  const bool row_in = g.qi < a.Lq;
  const bool row_ok = g.qi < g.q_hi;

  float qf[D / 2];
  {
    const float* qrow =
        (const float*)a.q + ((size_t)(g.b * a.Lq + (row_in ? g.qi : 0)) * a.Hq + g.h) * D + half * (D / 2);
#pragma unroll
    for (int s = 0; s < D / 8; ++s) {
      f32x4 r = {0.f, 0.f, 0.f, 0.f};
      if (row_in) r = *(const f32x4*)(qrow + 4 * s);
#pragma unroll
      for (int j = 0; j < 4; ++j) qf[4 * s + j] = r[j];
    }
  }
  const float* brow = nullptr;
  if constexpr (BIAS) {
    brow = a.bias + (size_t)g.b * a.bias_bstride + (size_t)g.h * a.bias_hstride +
           (size_t)(row_in ? g.qi : 0) * a.Lk;
  }
  const bool bias_vec = (a.Lk & 3) == 0;
  const float cx = (BIAS || EXT == 2) ? kLog2e : a.scale * kLog2e;
  ExtRows er;
  if constexpr (EXT > 0) er = ext_rows(a, g);

  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16{};
  float m_run = kMaxInit, l_run = 0.f;
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
      f32x4 rk = {0.f, 0.f, 0.f, 0.f}, rv = {0.f, 0.f, 0.f, 0.f};
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
      *(f32x4*)(&v_lds[buf][(u / DC) * VS + (u % DC) * 4]) = vreg[i];
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
    f32x16 s[BK / 32];
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb) {
      s[kb] = f32x16{};
      const float* kp = kl + (kb * 32 + col) * KS + half * (D / 2);
#pragma unroll
      for (int st4 = 0; st4 < D / 8; ++st4) {
        const f32x4 kf = *(const f32x4*)(kp + 4 * st4);
#pragma unroll
        for (int j = 0; j < 4; ++j) s[kb] = mfma32x32x2f32(kf[j], qf[4 * st4 + j], s[kb]);
      }
    }
    if constexpr (EXT == 2) {
      ext_scores_sT<BK / 32, BIAS>(a, g, er, s, k0, half, brow, row_in,
                                   [&](int kb, int r, float x, float) { s[kb][r] = x; });
    } else if constexpr (BIAS) {
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
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = xor32_max(mx);
    const float m_new = fmaxf(m_run, mx * cx);
    const float corr = fast_exp2(m_run - m_new);
    m_run = m_new;
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(s[kb][r], cx, -m_new));
        rs += p;
        s[kb][r] = p;
      }
    l_run = fmaf(l_run, corr, rs);
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] *= corr;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          acc[db] = mfma32x32x2f32(vl[key * VS + db * 32 + col], s[kb][r], acc[db]);
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

  const float l_tot = xor32_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row_in) {
    float* orow = (float*)a.o + ((size_t)(g.b * a.Lq + g.qi) * a.Hq + g.h) * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = acc[db][4 * gq + j] * inv;
        *(f32x4*)(orow + db * 32 + 8 * gq + 4 * half) = v;
      }
    if (a.lse && half == 0)
      a.lse[((size_t)g.b * a.Hq + g.h) * a.Lq + g.qi] =
          l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : INFINITY;
  }
}

// ---------------------------------------------------------------------------
// fp32, small grids: the key range of one 32-row query block is split over
// the 8 waves of a workgroup, so a problem with few query tiles still spreads
// over many SIMDs (the fp32 MFMA rate makes one wave's pass over all keys the
// critical path otherwise).  Wave w takes 32-key blocks w, w+NW, w+2NW, ...;
// each block's K half-rows and V columns are loaded from global memory
// straight into the MFMA operand registers (the next block's loads are in
// flight while one is computed), so no LDS staging is needed.  Each wave
// keeps its own online softmax; the partial (max, sum, O) are combined in LDS
// at the end.  NW = 8 waves for D = 64; D = 128 uses 4 (one per SIMD): its
// double-buffered operand blocks need more than the 256 registers of two
// waves per SIMD.  Products and softmax are those of flash_fwd_f32_kernel
// (v_mfma_f32_32x32x2f32, keys as MFMA rows).
// ---------------------------------------------------------------------------
template <int D>
constexpr int split_waves() { return D == 128 ? 4 : 8; }

template <int D, bool BIAS>
__global__ __launch_bounds__(64 * split_waves<D>(), 1) void flash_fwd_f32_split_kernel(FlashArgs a) {
  constexpr int NW = split_waves<D>();
  constexpr int DH = D / 2;          // floats per half row
  constexpr int OS = D + 4;          // combine row stride (floats)
  __shared__ __attribute__((aligned(16))) float red_o[NW * 32 * OS];
  __shared__ float red_ml[NW * 32 * 2];

  // Workgroup -> (32-row query block, batch, head); batch*head fastest.
  const int BH = a.B * a.Hq;
  const int bh = blockIdx.x % BH;
  const int qb = blockIdx.x / BH;
  const int b = bh / a.Hq, h = bh % a.Hq, hkv = h / (a.Hq / a.Hkv);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int qw = qb * 32;
  const int qi = qw + col;
  const int q_hi = min(a.Lq, a.q_valid);
  int kv_end = min(a.Lk, a.kv_valid);
  if (a.kv_lengths) kv_end = min(kv_end, max(a.kv_lengths[b], 0));
  int kv_stop = kv_end;
  if (qw >= q_hi) kv_stop = 0;
  else if (a.causal) kv_stop = min(kv_stop, min(qw + 32, q_hi));
  const int nkb = (kv_stop + 31) / 32;
  const bool row_in = qi < a.Lq;
  const bool row_ok = qi < q_hi;
  const size_t kv_row = (size_t)a.Hkv * D;
  const float* Kb = (const float*)a.k + ((size_t)b * a.Lk * a.Hkv + hkv) * D;
  const float* Vb = (const float*)a.v + ((size_t)b * a.Lk * a.Hkv + hkv) * D;

  float qf[DH];
  {
    const float* qrow = (const float*)a.q + ((size_t)(b * a.Lq + (row_in ? qi : 0)) * a.Hq + h) * D + half * DH;
#pragma unroll
    for (int s = 0; s < DH / 4; ++s) {
      f32x4 r = {0.f, 0.f, 0.f, 0.f};
      if (row_in) r = *(const f32x4*)(qrow + 4 * s);
#pragma unroll
      for (int j = 0; j < 4; ++j) qf[4 * s + j] = r[j];
    }
  }
  const float* brow = nullptr;
  if constexpr (BIAS)
    brow = a.bias + (size_t)b * a.bias_bstride + (size_t)h * a.bias_hstride + (size_t)(row_in ? qi : 0) * a.Lk;
  const bool bias_vec = (a.Lk & 3) == 0;
  const float cx = BIAS ? kLog2e : a.scale * kLog2e;

  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16{};
  float m_run = kMaxInit, l_run = 0.f;

  // Operand registers of one 32-key block: K half row of key k0 + col (dims
  // half*D/2 + [0, D/2)); V column db*32 + col at the 16 keys of slot r
  // (key k0 + 8*(r/4) + 4*half + r%4).  Keys at or past kv_stop read 0.
  struct Block {
    float k[DH];
    float v[D / 32][16];
  };
  auto load = [&](int kbk, Block& blk) {
    const int k0 = kbk * 32;
    const int kk = k0 + col;
    const bool kin = kbk < nkb && kk < kv_stop;
    const float* kp = Kb + (size_t)(kin ? kk : 0) * kv_row + half * DH;
#pragma unroll
    for (int s = 0; s < DH / 4; ++s) {
      f32x4 r = {0.f, 0.f, 0.f, 0.f};
      if (kin) r = *(const f32x4*)(kp + 4 * s);
#pragma unroll
      for (int j = 0; j < 4; ++j) blk.k[4 * s + j] = r[j];
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
      const bool vin = kbk < nkb && key < kv_stop;
      const float* vp = Vb + (size_t)(vin ? key : 0) * kv_row + col;
#pragma unroll
      for (int db = 0; db < D / 32; ++db) blk.v[db][r] = vin ? vp[db * 32] : 0.f;
    }
  };
  auto compute = [&](int kbk, const Block& blk) {
    const int k0 = kbk * 32;
    f32x16 s = f32x16{};
#pragma unroll
    for (int st = 0; st < DH; ++st) s = mfma32x32x2f32(blk.k[st], qf[st], s);
    if constexpr (BIAS) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int kk = k0 + 8 * gq + 4 * half;
        f32x4 bv = {0.f, 0.f, 0.f, 0.f};
        if (row_in) bv = bias_vec ? load_bias4<true>(brow, kk, a.Lk) : load_bias4<false>(brow, kk, a.Lk);
#pragma unroll
        for (int j = 0; j < 4; ++j) s[4 * gq + j] = fmaf(s[4 * gq + j], a.scale, bv[j]);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
      const bool keep = row_ok && kk < kv_end && (!a.causal || kk <= qi);
      if (!keep) s[r] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
    mx = xor32_max(mx);
    const float m_new = fmaxf(m_run, mx * cx);
    const float corr = fast_exp2(m_run - m_new);
    m_run = m_new;
    float rs = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(fmaf(s[r], cx, -m_new));
      rs += p;
      s[r] = p;
    }
    l_run = fmaf(l_run, corr, rs);
#pragma unroll
    for (int i = 0; i < D / 32; ++i) acc[i] *= corr;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[db] = mfma32x32x2f32(blk.v[db][r], s[r], acc[db]);
  };

  // This wave's blocks w, w+NW, ... (a wave may have none: it then combines
  // an empty partial).
  Block cur, nxt;
  load(w, cur);
  for (int kbk = w; kbk < nkb; kbk += NW) {
    load(kbk + NW, nxt);
    compute(kbk, cur);
    cur = nxt;
  }

  // ---- combine the NW partials in LDS ----
  l_run = xor32_sum(l_run);
  {
    float* ro = red_o + (size_t)w * 32 * OS;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
        *(f32x4*)(ro + col * OS + db * 32 + 8 * gq + 4 * half) =
            f32x4{acc[db][4 * gq], acc[db][4 * gq + 1], acc[db][4 * gq + 2], acc[db][4 * gq + 3]};
    if (half == 0) {
      red_ml[(w * 32 + col) * 2] = m_run;
      red_ml[(w * 32 + col) * 2 + 1] = l_run;
    }
  }
  __syncthreads();
  constexpr int NQ = D / 4;
  for (int idx = tid; idx < 32 * NQ; idx += 64 * NW) {
    const int r = idx / NQ, u = idx % NQ;
    const int q = qw + r;
    float M = kMaxInit;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, red_ml[(ww * 32 + r) * 2]);
    float L = 0.f;
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float wt = fast_exp2(red_ml[(ww * 32 + r) * 2] - M);
      L = fmaf(wt, red_ml[(ww * 32 + r) * 2 + 1], L);
      O += wt * *(const f32x4*)(red_o + (size_t)(ww * 32 + r) * OS + 4 * u);
    }
    if (q < a.Lq) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      *(f32x4*)((float*)a.o + ((size_t)(b * a.Lq + q) * a.Hq + h) * D + 4 * u) = O * inv;
      if (a.lse && u == 0)
        a.lse[((size_t)b * a.Hq + h) * a.Lq + q] = L > 0.f ? (M + __log2f(L)) * kLn2 : INFINITY;
    }
  }
}

template <auto K>
static int launch(const FlashArgs& a, hipStream_t stream, int threads = kThreads) {
  const long blocks = (long)a.n_qtiles * a.B * a.Hq;
  launch_kernel<K>(dim3((unsigned)blocks), dim3(threads), 0, stream, a);
  return check_launch("pjx_flash_fwd");
}

// The pipelined bf16 kernel at D = 128: 32-key tiles (3 workgroups per CU)
// when the grid fills at least one round of them; smaller grids (one round of
// 2 per CU or less, as at batch*heads = 16) run 64-key tiles, whose longer
// steps between barriers hide latency better at that occupancy (measured:
// 87 us against 113 us at B=1, H=16, L=4096 causal; 1-1.5% slower than
// 32-key tiles from 1024 workgroups up).  Grids of at most one workgroup per
// CU (two, causal) run the two-group form: 81 against 89 us there.
template <typename E>
static int launch_pipe128(const FlashArgs& a, hipStream_t stream) {
  const int cus = device_cu_count();
  const long blocks = (long)a.n_qtiles * a.B * a.Hq;
  if (blocks <= 2L * cus && (a.causal || blocks <= cus))
    return launch<flash_fwd_bf16_pipe_kernel<E, 128, 64, 2, 2>>(a, stream, 2 * kThreads);
  if (blocks < 3L * cus) return launch<flash_fwd_bf16_pipe_kernel<E, 128, 64, 2>>(a, stream);
  return launch<flash_fwd_bf16_pipe_kernel<E, 128, 32, 3>>(a, stream);
}

// The 16-bit kernels (bf16 or fp16 operands, format E) for head_dim 64 / 128.
template <typename E>
static int launch_h16(const FlashArgs& a, int head_dim, hipStream_t s) {
  const bool hb = a.bias != nullptr;
  if (a.ext) {
    // Extended masks / score modifiers: the one-pass kernel's EXT variants
    // (1: interval masks, 2: segment ids / score modifiers as well).
    const bool full = a.ext == 2;
    if (head_dim == 128) {
      if (full) return hb ? launch<flash_fwd_bf16_kernel<E, 128, true, 2>>(a, s) : launch<flash_fwd_bf16_kernel<E, 128, false, 2>>(a, s);
      return hb ? launch<flash_fwd_bf16_kernel<E, 128, true, 1>>(a, s) : launch<flash_fwd_bf16_kernel<E, 128, false, 1>>(a, s);
    }
    if (full) return hb ? launch<flash_fwd_bf16_kernel<E, 64, true, 2>>(a, s) : launch<flash_fwd_bf16_kernel<E, 64, false, 2>>(a, s);
    return hb ? launch<flash_fwd_bf16_kernel<E, 64, true, 1>>(a, s) : launch<flash_fwd_bf16_kernel<E, 64, false, 1>>(a, s);
  }
  // Dense bias with 16-byte aligned rows and 32-bit slice offsets: the LDS
  // ring that streams the bias; otherwise bias loads into registers.
  const bool ring = hb && a.Lk % 4 == 0 && (int64_t)a.Lq * a.Lk * 4 < ((int64_t)1 << 31);
  if (head_dim == 128) {
    if (ring) return launch_flash_bias_ring(128, a, s);
    return hb ? launch<flash_fwd_bf16_kernel<E, 128, true, 0>>(a, s) : launch_pipe128<E>(a, s);
  }
  if (ring) return launch_flash_bias_ring(64, a, s);
  if (hb) return launch<flash_fwd_bf16_kernel<E, 64, true, 0>>(a, s);
  const long blocks = (long)a.n_qtiles * a.B * a.Hq;
  const int cus = device_cu_count();
  if (blocks <= 2L * cus && (a.causal || blocks <= cus))
    return launch<flash_fwd_bf16_pipe_kernel<E, 64, 64, 2, 2>>(a, s, 2 * kThreads);
  return launch<flash_fwd_bf16_pipe_kernel<E, 64, 64, 2>>(a, s);
}

// The fp32 split kernel: one workgroup per 32-row query block.
template <int D, auto K>
static int launch_split(const FlashArgs& a, hipStream_t stream) {
  const long blocks = (long)((a.Lq + 31) / 32) * a.B * a.Hq;
  if (blocks > 0x7fffffffL) return fail(PJX_ERR_INVALID, "pjx_flash_fwd: grid too large");
  launch_kernel<K>(dim3((unsigned)blocks), dim3(64 * split_waves<D>()), 0, stream, a);
  return check_launch("pjx_flash_fwd");
}

}  // namespace pjx

using namespace pjx;

// Checks the arguments shared by pjx_flash_fwd and pjx_mla_fwd and fills the
// argument block; returns PJX_OK, or an error (message set).  *empty is set
// when there is nothing to compute.
static int make_flash_args(FlashArgs& a, const char* who, const void* q, const void* k,
                           const void* v, void* o, float* lse, const int32_t* kv_lengths,
                           const float* bias, int64_t bias_batch, int64_t bias_heads, int64_t batch,
                           int64_t q_len, int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                           int64_t head_dim, int64_t v_dim, int64_t q_valid, int64_t kv_valid,
                           int causal, float sm_scale, const pjx_score_mods* mods, bool* empty) {
  char buf[256];
  *empty = false;
  // zero-element tensors may come as null pointers
  const bool q_none = batch == 0 || q_len == 0, k_none = batch == 0 || kv_len == 0;
  if ((!q_none && (!q || !o)) || (!k_none && (!k || !v))) {
    snprintf(buf, sizeof(buf), "%s: input and output pointers must be non-null", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  if (batch < 0 || q_len < 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0) {
    snprintf(buf, sizeof(buf), "%s: negative or zero size", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  if (q_heads % kv_heads != 0) {
    snprintf(buf, sizeof(buf), "%s: q_heads must be a multiple of kv_heads", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  if (!(sm_scale > 0.f)) {
    snprintf(buf, sizeof(buf), "%s: sm_scale must be > 0", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  if (bias && !((bias_batch == 1 || bias_batch == batch) && (bias_heads == 1 || bias_heads == q_heads))) {
    snprintf(buf, sizeof(buf), "%s: bias must be [1|B, 1|Hq, Lq, Lk]", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  const int64_t elems = batch * q_len * q_heads * std::max(head_dim, v_dim);
  if (elems > (int64_t)1 << 40 || q_len > (1 << 30) || kv_len > (1 << 30) ||
      kv_len * kv_heads * head_dim * 2 > ((int64_t)1 << 40)) {
    snprintf(buf, sizeof(buf), "%s: sizes out of range", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  if (batch == 0 || q_len == 0) {
    *empty = true;
    return PJX_OK;
  }
  a.q = q; a.k = k; a.v = v; a.o = o; a.lse = lse;
  a.kv_lengths = kv_lengths;
  a.bias = bias;
  a.bias_hstride = (bias && bias_heads != 1) ? q_len * kv_len : 0;
  a.bias_bstride = (bias && bias_batch != 1) ? bias_heads * q_len * kv_len : 0;
  a.B = (int)batch; a.Lq = (int)q_len; a.Lk = (int)kv_len;
  a.Hq = (int)q_heads; a.Hkv = (int)kv_heads;
  a.q_valid = (int)std::min<int64_t>(std::max<int64_t>(q_valid, 0), q_len);
  a.kv_valid = (int)std::min<int64_t>(std::max<int64_t>(kv_valid, 0), kv_len);
  a.causal = causal ? 1 : 0;
  a.f16 = 0;
  a.scale = sm_scale;
  a.n_qtiles = (int)((q_len + kBQ - 1) / kBQ);
  a.dv = (int)v_dim;
  if ((long)a.n_qtiles * batch * q_heads > 0x7fffffffL) {
    snprintf(buf, sizeof(buf), "%s: grid too large", who);
    return fail(PJX_ERR_INVALID, buf);
  }
  return lower_score_mods(mods, a, who);
}

extern "C" int pjx_flash_fwd(int dtype, const void* q, const void* k, const void* v, void* o,
                             float* lse, const int32_t* kv_lengths, const float* bias,
                             int64_t bias_batch, int64_t bias_heads, int64_t batch,
                             int64_t q_len, int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                             int64_t head_dim, int64_t q_valid, int64_t kv_valid, int causal,
                             float sm_scale, const pjx_score_mods* mods, void* stream) {
  clear_error();
  if (dtype != PJX_DTYPE_BF16 && dtype != PJX_DTYPE_F16 && dtype != PJX_DTYPE_F32)
    return fail(PJX_ERR_INVALID, "pjx_flash_fwd: dtype must be PJX_DTYPE_BF16, PJX_DTYPE_F16 or PJX_DTYPE_F32");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(PJX_ERR_INVALID, "pjx_flash_fwd: head_dim must be 64, 128 or 256");
  FlashArgs a;
  bool empty;
  int rc = make_flash_args(a, "pjx_flash_fwd", q, k, v, o, lse, kv_lengths, bias, bias_batch,
                           bias_heads, batch, q_len, kv_len, q_heads, kv_heads, head_dim, head_dim,
                           q_valid, kv_valid, causal, sm_scale, mods, &empty);
  if (rc != PJX_OK || empty) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (kv_len == 0)
    return write_keyless(o, lse, (size_t)(batch * q_len * q_heads * head_dim), dtype == PJX_DTYPE_F32,
                         (size_t)(batch * q_heads * q_len), s, "pjx_flash_fwd");
  const bool hb = bias != nullptr;
  a.f16 = dtype == PJX_DTYPE_F16;
  if (head_dim == 256) return dtype == PJX_DTYPE_F32 ? launch_flash_f32_wide(a, s) : launch_flash_wide256(a, s);
  if (dtype == PJX_DTYPE_BF16) return launch_h16<Bf16Fmt>(a, (int)head_dim, s);
  if (dtype == PJX_DTYPE_F16) return launch_h16<F16Fmt>(a, (int)head_dim, s);
  if (a.ext) {
    const bool full = a.ext == 2;
    if (head_dim == 128) {
      if (full) return hb ? launch<flash_fwd_f32_kernel<128, true, 2>>(a, s) : launch<flash_fwd_f32_kernel<128, false, 2>>(a, s);
      return hb ? launch<flash_fwd_f32_kernel<128, true, 1>>(a, s) : launch<flash_fwd_f32_kernel<128, false, 1>>(a, s);
    }
    if (full) return hb ? launch<flash_fwd_f32_kernel<64, true, 2>>(a, s) : launch<flash_fwd_f32_kernel<64, false, 2>>(a, s);
    return hb ? launch<flash_fwd_f32_kernel<64, true, 1>>(a, s) : launch<flash_fwd_f32_kernel<64, false, 1>>(a, s);
  }
  // fp32 with fewer 128-row workgroups than CUs: split each query block's
  // keys over several waves (latency-bound sizes, like the reference's CPU
  // case).
  if ((long)a.n_qtiles * batch * q_heads < 256) {
    if (head_dim == 128)
      return hb ? launch_split<128, flash_fwd_f32_split_kernel<128, true>>(a, s)
                : launch_split<128, flash_fwd_f32_split_kernel<128, false>>(a, s);
    return hb ? launch_split<64, flash_fwd_f32_split_kernel<64, true>>(a, s)
              : launch_split<64, flash_fwd_f32_split_kernel<64, false>>(a, s);
  }
  if (head_dim == 128) return hb ? launch<flash_fwd_f32_kernel<128, true, 0>>(a, s) : launch<flash_fwd_f32_kernel<128, false, 0>>(a, s);
  return hb ? launch<flash_fwd_f32_kernel<64, true, 0>>(a, s) : launch<flash_fwd_f32_kernel<64, false, 0>>(a, s);
}

extern "C" int pjx_mla_fwd(int dtype, const void* q, const void* cache, void* o, float* lse,
                           const int32_t* kv_lengths, const float* bias, int64_t bias_batch,
                           int64_t bias_heads, int64_t batch, int64_t q_len, int64_t kv_len,
                           int64_t heads, int64_t rank, int64_t v_dim, int64_t q_valid,
                           int64_t kv_valid, int causal, float sm_scale,
                           const pjx_score_mods* mods, void* stream) {
  clear_error();
  if (dtype != PJX_DTYPE_BF16 && dtype != PJX_DTYPE_F16)
    return fail(PJX_ERR_INVALID, "pjx_mla_fwd: dtype must be PJX_DTYPE_BF16 or PJX_DTYPE_F16");
  const bool wide = (rank == 576 && (v_dim == 512 || v_dim == 576)) || (rank == 512 && v_dim == 512);
  const bool narrow = (rank == 64 || rank == 128 || rank == 256) && v_dim == rank;
  if (!wide && !narrow)
    return fail(PJX_ERR_INVALID,
                "pjx_mla_fwd: (rank, v_dim) must be (576, 512), (576, 576), (512, 512) or rank in "
                "{64, 128, 256} with v_dim == rank");
  if (narrow)  // the latent as one shared K = V head of the flash kernels
    return pjx_flash_fwd(dtype, q, cache, cache, o, lse, kv_lengths, bias, bias_batch, bias_heads,
                         batch, q_len, kv_len, heads, 1, rank, q_valid, kv_valid, causal, sm_scale,
                         mods, stream);
  FlashArgs a;
  bool empty;
  int rc = make_flash_args(a, "pjx_mla_fwd", q, cache, cache, o, lse, kv_lengths, bias, bias_batch,
                           bias_heads, batch, q_len, kv_len, heads, 1, rank, v_dim, q_valid,
                           kv_valid, causal, sm_scale, mods, &empty);
  if (rc != PJX_OK || empty) return rc;
  if (kv_len == 0)
    return write_keyless(o, lse, (size_t)(batch * q_len * heads * v_dim), false, (size_t)(batch * heads * q_len),
                         (hipStream_t)stream, "pjx_mla_fwd");
  a.f16 = dtype == PJX_DTYPE_F16;
  return launch_mla_wide(a, (int)rank, (hipStream_t)stream);
}
