// Flash-attention forward for wide heads on gfx950 (MI355X), bf16 or fp16: head dims
// above 128 (D = 256) and the absorbed latent attention of probjax's `mla`
// (K = V = one shared latent row of R = 512 or 576 values per key, Hkv = 1;
// probjax/nn/pallas_kernels/kernels/latent_attention.py:79-197, 636-766).
//
// Semantics are those of flash_fwd.hip (the XLA reference,
// kernels/attention_xla.py:339-429): s = sm_scale * q.k in fp32, then the
// bias, then the mask (-inf), online softmax in the exp2 domain, P rounded to
// the input's 16-bit format before P.V, fp32 accumulation, rows without a valid key give 0.
//
// Decomposition: one workgroup = 4 waves = 128 query rows of one (batch,
// head), 32 rows per wave, as in flash_fwd.hip.  S^T = K Q^T puts the keys on
// the rows of v_mfma_f32_32x32x16_bf16 (one query per lane: lane-local row
// max and sum); O^T += V^T P^T takes P straight from registers.  A wave holds
// Q^T for all D dims (D/4 VGPRs: 144 at D = 576) and O^T for DVP output dims
// (DVP/2 accumulators: 256 at DVP = 512): at D = 256 without bias or extended
// masks two waves fit a SIMD (measured 406 -> 263 us on a B=2, H=16, L=4096
// causal forward against one wave), otherwise one runs per SIMD.
// Output widths above 256 (the latent's 512, or the API-exact 576 of an
// R = 576 latent) are split into parts of DVP dims: the grid carries one
// workgroup per part of each (q tile, batch, head), adjacent in launch order so
// that both read the same K/V tiles through L2, and each forms the whole score
// for its rows.  (Q^T, O^T for all 512 dims and the score would need more
// than the 512 registers a wave has here.)
//
// Data movement: the K/V tile of BK keys goes HBM -> LDS with buffer loads
// that write LDS directly; with SHARED (the latent) one tile serves both
// products: its rows are the keys, its first DV columns the values, read once
// from HBM and twice from LDS.  Two stages; the next tile's loads are in
// flight while one is computed.
//
// LDS row layout: row-major [key][dim] rows of 2D bytes whose 16-byte chunks
// are XOR-swizzled within aligned groups of G chunks by a function of the row.
// One swizzle serves both read patterns:
//   * K fragments (ds_read_b128): 16 lanes read one chunk of 16 consecutive
//     rows;
//   * V^T fragments (ds_read_b64_tr_b16): 32 lanes read 4 chunks of 4
//     consecutive rows (starting at a multiple of 4).
// With rows a whole number of 256-byte bank lines (D = 128, 256, 512; G = 16)
// every row starts at bank 0 and swz(r) = 4(r&3) + ((r>>2)&3) is a bijection on
// any 16 consecutive rows that puts 4 consecutive rows in 4 different 4-chunk
// blocks.  With rows of an odd number of half lines (D = 192, 576; G = 8) odd
// rows start half a line later; swz(r) = 4((r>>1)&1) + ((r>>2)&3) is then a
// bijection on the 8 rows of each parity among 16 consecutive rows, and puts
// rows r and r+2 in different 4-chunk blocks.
#include "flash_common.h"

namespace pjx {

template <int D>
struct WideRow {
  static constexpr int ROWB = 2 * D;  // bytes per row
  static constexpr int NC = D / 8;    // 16-byte chunks per row
  static constexpr bool FULL_LINES = (ROWB % 256) == 0;
  static constexpr int G = FULL_LINES ? 16 : 8;  // swizzle group (chunks)
  static_assert(ROWB % 256 == 0 || ROWB % 256 == 128, "rows of whole or half bank lines");
  static_assert(NC % G == 0, "rows of whole swizzle groups");
  __device__ static int swz(int r) {
    return FULL_LINES ? 4 * (r & 3) + ((r >> 2) & 3) : 4 * ((r >> 1) & 1) + ((r >> 2) & 3);
  }
};

// Waves per SIMD: two where the kernel fits 256 registers without spilling
// (D = 256 without bias or extended masks: 242 VGPRs), else one.
template <int D, bool BIAS, int EXT>
constexpr int wide_fwd_occupancy() { return (D <= 256 && !BIAS && EXT == 0) ? 2 : 1; }

template <typename E, int D, int DVP, int BK, bool SHARED, bool BIAS, int EXT>
__global__ __launch_bounds__(kThreads, (wide_fwd_occupancy<D, BIAS, EXT>())) void flash_fwd_wide_kernel(FlashArgs a) {
  using R = WideRow<D>;
  constexpr int ROWB = R::ROWB, NC = R::NC, G = R::G;
  constexpr int TILE_B = BK * ROWB;                  // one tensor's tile
  constexpr int STAGE_B = SHARED ? TILE_B : 2 * TILE_B;
  constexpr int UNITS = BK * NC;                     // 16-byte units per tile
  static_assert(UNITS % 256 == 0, "a tile splits into whole 1 KiB wave loads");
  constexpr int NLD = UNITS / 256;                   // loads per wave per tensor
  constexpr int KS = D / 16;                         // 16-dim steps of Q.K
  constexpr int NDB = DVP / 32;                      // 32-dim output blocks
  constexpr int KE = G / 2;                          // distinct K-fragment offsets
  constexpr int VE = G / 4;                          // V^T-fragment offsets (period in db)
  static_assert(BK % 32 == 0 && DVP % 32 == 0 && DVP <= D, "tile shapes");
  __shared__ __attribute__((aligned(1024))) unsigned char smem0[STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char smem1[STAGE_B];

  // Output part (dims dv_off .. dv_off + DVP) and (q tile, batch, head).
  const int n_parts = a.dv / DVP;
  const int part = (int)blockIdx.x % n_parts;
  const int dv_off = part * DVP;
  BlockGeom g = block_geom(a, (int)blockIdx.x / n_parts);
  if constexpr (EXT > 0) ext_block_range(a, g, BK);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  g.qw = __builtin_amdgcn_readfirstlane(g.qw);
  const int col = lane & 31, half = lane >> 5;
  const uint32_t rowstride = (uint32_t)a.Hkv * ROWB;
  const unsigned char* Kb = (const unsigned char*)a.k + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * ROWB;
  const unsigned char* Vb = (const unsigned char*)a.v + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * ROWB;
  const bool row_in = g.qi < a.Lq;
  const bool row_ok = g.qi < g.q_hi;

  // Q^T as the B operand: lane holds query `col`, dims 16*st + 8*half + [0,8).
  typename E::v8 qf[KS];
  {
    const uint16_t* qrow =
        (const uint16_t*)a.q + ((size_t)(g.b * a.Lq + (row_in ? g.qi : 0)) * a.Hq + g.h) * D;
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row_in) raw = *(const u32x4*)(qrow + 16 * st + 8 * half);
      qf[st] = E::as8(raw);
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

  // Buffer->LDS sources: load j of wave w fills 16-byte unit
  // p = (NLD*w + j)*64 + lane = row*NC + slot of the tile, from global
  // chunk slot ^ swz(row) of that row.
  uint32_t voff[NLD];
#pragma unroll
  for (int j = 0; j < NLD; ++j) {
    const int p = (NLD * w + j) * 64 + lane, r = p / NC, slot = p % NC;
    voff[j] = r * rowstride + 16 * (slot ^ R::swz(r));
  }
  // K fragment of step st: row `col` of a 32-key block, chunk 2*st + half,
  // i.e. group st / KE, chunk 2*(st % KE) + half within it.
  uint32_t offK[KE];
#pragma unroll
  for (int e = 0; e < KE; ++e) offK[e] = col * ROWB + 16 * ((2 * e + half) ^ R::swz(col));
  // V^T fragment of output block db, 16-key step c: lane s16 of 16-lane group
  // grp reads row 16c + 4*half + s16/4 (+8 for the second read), bytes
  // 8*(s16&1) of chunk ch + 2*(grp&1) + ((s16&3)>>1), ch = dv_off/8 + 4*db.
  // Writing db = VE*i + j (j < VE), chunk ch lies in swizzle group
  // (dv_off/8 + 4j)/G + i at position (dv_off/8 + 4j) % G: the address is
  // base[j] + 16*G*i with VE per-lane bases fixed for the kernel.
  uint32_t offVlo[VE], offVhi[VE];
  {
    const int s16 = lane & 15, grp = lane >> 4;
    const int low = 2 * (grp & 1) + ((s16 & 3) >> 1);
    const int rl = 4 * half + (s16 >> 2), rh = rl + 8;
    const int c0 = dv_off / 8;
#pragma unroll
    for (int j = 0; j < VE; ++j) {
      const int ch = c0 + 4 * j, grp_ofs = 16 * G * (ch / G), pos = ch % G;
      offVlo[j] = grp_ofs + rl * ROWB + 16 * ((pos + low) ^ R::swz(rl)) + 8 * (s16 & 1);
      offVhi[j] = grp_ofs + rh * ROWB + 16 * ((pos + low) ^ R::swz(rh)) + 8 * (s16 & 1);
    }
  }

  f32x16 acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc[i] = f32x16{};
  float m_run = kMaxInit, l_run = 0.f;

  const int t_begin = g.kv_begin / BK;
  const int n_tiles = max((g.kv_stop + BK - 1) / BK - t_begin, 0);
  const int q_last_w = g.qw + 31;

  auto issue = [&](int t, unsigned char* st) {
    const int k0 = (t_begin + t) * BK;
    const int nvalid = min(BK, g.kv_stop - k0);
    const uint32_t bytes = (uint32_t)(nvalid - 1) * rowstride + ROWB;
    const rsrc_t rk = make_rsrc(Kb + (size_t)k0 * rowstride, bytes);
#pragma unroll
    for (int j = 0; j < NLD; ++j) buffer_load_lds16(rk, st + (NLD * w + j) * 1024, voff[j]);
    if constexpr (!SHARED) {
      const rsrc_t rv = make_rsrc(Vb + (size_t)k0 * rowstride, bytes);
#pragma unroll
      for (int j = 0; j < NLD; ++j) buffer_load_lds16(rv, st + TILE_B + (NLD * w + j) * 1024, voff[j]);
    }
  };

  auto compute = [&](int t, const unsigned char* ks) {
    const int k0 = (t_begin + t) * BK;
    if constexpr (EXT > 0) {
      if (!er.any || k0 > er.hi_last || k0 + BK - 1 < er.lo_first) return;
    } else {
      if (a.causal && k0 > q_last_w) return;  // tile above this wave's diagonal
    }
    const unsigned char* vs = SHARED ? ks : ks + TILE_B;

    // S^T[key][query] = K Q^T
    f32x16 s[BK / 32];
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb) {
      s[kb] = f32x16{};
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        const typename E::v8 kf =
            E::as8(*(const u32x4*)(ks + kb * 32 * ROWB + 16 * G * (st / KE) + offK[st % KE]));
        s[kb] = E::mma32(kf, qf[st], s[kb]);
      }
    }
    // K-fragment reads 3 MFMAs ahead (left to itself the scheduler, at these
    // register counts, waits for each read right before its MFMA: measured
    // 17% slower on the latent prefill, 2.6% on D = 256).
    PJX_SCHED_LDS_READS_AHEAD(KS * (BK / 32), 3, 1);

    // Register r of block kb holds key k0 + kb*32 + 8*(r/4) + 4*half + r%4.
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
      for (int i = 0; i < NDB; ++i)
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
    // O^T[d][query] += V^T P^T: output block db covers chunks dv_off/8 + 4*db + [0,4).
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int gofs = 16 * G * (db / VE);
      const int e = db % VE;
#pragma unroll
      for (int c = 0; c < BK / 16; ++c) {
        const u32x2 lo = lds_read_tr16(vs + 16 * c * ROWB + gofs + offVlo[e]);
        const u32x2 hi = lds_read_tr16(vs + 16 * c * ROWB + gofs + offVhi[e]);
        const u32x4 av = {lo[0], lo[1], hi[0], hi[1]};
        acc[db] = E::mma32(E::as8(av), pf[c], acc[db]);
      }
    }
  };

  // Tile t lives in stage t % 2 (the protocol of flash_fwd.hip's one-pass
  // kernel): this wave's loads of tile t have landed (waitcnt), then every
  // wave's have and every wave is done with the other stage (barrier), so
  // tile t+1's loads go there while tile t is computed.
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
    uint16_t* orow = (uint16_t*)a.o + ((size_t)(g.b * a.Lq + g.qi) * a.Hq + g.h) * a.dv + dv_off;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        u32x2 pk;
        pk[0] = E::pack2(acc[db][4 * gq] * inv, acc[db][4 * gq + 1] * inv);
        pk[1] = E::pack2(acc[db][4 * gq + 2] * inv, acc[db][4 * gq + 3] * inv);
        *(u32x2*)(orow + db * 32 + 8 * gq + 4 * half) = pk;
      }
    if (part == 0 && a.lse && half == 0)
      a.lse[((size_t)g.b * a.Hq + g.h) * a.Lq + g.qi] =
          l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : INFINITY;
  }
}

template <auto K>
static int launch_wide(const FlashArgs& a, int n_parts, hipStream_t stream, const char* who) {
  const long blocks = (long)a.n_qtiles * a.B * a.Hq * n_parts;
  if (blocks > 0x7fffffffL) return fail(PJX_ERR_INVALID, "wide flash forward: grid too large");
  launch_kernel<K>(dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  return check_launch(who);
}

// One (D, DVP, BK, SHARED) shape over the bias / extended-mask variants.
// Interval masks (EXT = 1) run the full extended kernel: at these head widths
// the per-score mask work is a small share of the tile.
template <typename E, int D, int DVP, int BK, bool SHARED>
static int launch_wide_fmt(const FlashArgs& a, hipStream_t s, const char* who) {
  const int np = a.dv / DVP;
  const bool hb = a.bias != nullptr;
  if (a.ext)
    return hb ? launch_wide<flash_fwd_wide_kernel<E, D, DVP, BK, SHARED, true, 2>>(a, np, s, who)
              : launch_wide<flash_fwd_wide_kernel<E, D, DVP, BK, SHARED, false, 2>>(a, np, s, who);
  return hb ? launch_wide<flash_fwd_wide_kernel<E, D, DVP, BK, SHARED, true, 0>>(a, np, s, who)
            : launch_wide<flash_fwd_wide_kernel<E, D, DVP, BK, SHARED, false, 0>>(a, np, s, who);
}

template <int D, int DVP, int BK, bool SHARED>
static int launch_wide_variant(const FlashArgs& a, hipStream_t s, const char* who) {
  static_assert(DVP % 32 == 0, "parts of whole output blocks");
  if (a.dv % DVP != 0) return fail(PJX_ERR_INVALID, "wide flash forward: output width not a multiple of the part");
  return a.f16 ? launch_wide_fmt<F16Fmt, D, DVP, BK, SHARED>(a, s, who)
               : launch_wide_fmt<Bf16Fmt, D, DVP, BK, SHARED>(a, s, who);
}

// D = 256 flash forward (separate K and V), called by pjx_flash_fwd.
int launch_flash_wide256(FlashArgs& a, hipStream_t s) {
  a.dv = 256;
  return launch_wide_variant<256, 256, 32, false>(a, s, "pjx_flash_fwd");
}

// Absorbed latent forward: K = V = the latent rows (a.k == a.v, Hkv = 1),
// head dim `rank`, output width a.dv.
int launch_mla_wide(FlashArgs& a, int rank, hipStream_t s) {
  const char* who = "pjx_mla_fwd";
  if (rank == 576 && a.dv == 512) return launch_wide_variant<576, 256, 32, true>(a, s, who);
  if (rank == 576 && a.dv == 576) return launch_wide_variant<576, 288, 32, true>(a, s, who);
  if (rank == 512 && a.dv == 512) return launch_wide_variant<512, 256, 32, true>(a, s, who);
  return fail(PJX_ERR_INVALID, "pjx_mla_fwd: (rank, v_dim) must be (576, 512), (576, 576) or (512, 512)");
}

}  // namespace pjx
