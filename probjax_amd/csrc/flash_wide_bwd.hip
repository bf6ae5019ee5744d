// Flash-attention backward for wide heads on gfx950 (MI355X), bf16 or fp16: D = 256,
// and the absorbed latent of probjax's `mla` (K = V = one shared latent row of
// R = 512 or 576 values per key, Hkv = 1, output width DV <= R).
//
// probjax differentiates absorbed `mla` through the materialised computation
// (kernels/latent_attention.py:752-766): `mha` over K = V = the latent
// broadcast to every head, so the cache gradient is the sum over heads of
// dK + dV.  The math is the flash backward's (flash_bwd_kernels.h; probjax
// attention.py:853-1160): delta = sum_d o*do, p = exp2(s*log2e - lse*log2e),
// ds = p (do.v^T - delta) sm_scale, dq = sum_k r(ds) k,
// dk = sum_q r(ds)^T q, dv = sum_q r(p)^T do, fp32 accumulation (r() rounds
// to the input's 16-bit format).
//
// At these widths a wave cannot hold 32 rows of Q^T and dO^T and a 32-row dQ
// accumulator (1.5 K registers at R = 576), so both kernels put 16 rows (or
// 16 keys) on each wave and use v_mfma_f32_16x16x32_bf16:
//   A lane l holds A[l%16][8*(l/16) + j], B lane l holds B[8*(l/16) + j][l%16],
//   C register r of lane l is C[4*(l/16) + r][l%16].
// Writing c = l%16 and qd = l/16:
//   wide_bwd_dq_kernel -- one workgroup per (64-query tile, batch, head); a wave
//     owns rows qw + c.  K (and V) tiles of 32 keys stream HBM -> LDS.
//     S^T = K Q^T and dP^T = V dO^T (keys on the MFMA rows, so register r of
//     block kb is key k0 + 16kb + 4qd + r of the lane's row); with the shared
//     latent one K-fragment read feeds both products.  dQ^T += K^T dS^T takes
//     dS^T from registers as the B operand (k slot 8qd + j <-> key
//     16(j/4) + 4qd + j%4) and K^T from transposing LDS reads in that key
//     order.  It writes delta * sm_scale and lse*log2e for the second kernel.
//   wide_bwd_dkdv_kernel -- one workgroup per (64-key tile, batch, KV head,
//     head group); a wave owns keys kw + c with K^T (and V^T) in registers.
//     Q and dO tiles of 32 rows stream through LDS.  S = Q K^T, dP = dO V^T
//     (rows on the MFMA rows), then dK^T += Q^T dS and dV^T += dO^T P with
//     Q^T / dO^T from transposing reads.  With the shared latent both land in
//     one accumulator (dC = dK + dV).  A KV head's query heads are split into
//     groups over workgroups when one group per head-tile would leave the chip
//     idle (MQA: 16 heads over one latent); each group writes an fp32 partial
//     and wide_bwd_reduce_kernel sums them in a fixed order (deterministic).
//   wide_bwd_dc_kernel -- the same workgroup and outputs as the dK/dV kernel
//     for inputs without bias or extended masks, with the gradient update
//     split over the waves by columns instead of keys (P and dS exchanged
//     through LDS), so each wave reads a quarter of the transposed Q / dO
//     fragments.  The C-ABI reaches it for the latent; pjx_flash_bwd takes
//     D = 256 dK/dV without extended masks from its own 32-key kernel.
//
// LDS rows are row-major [row][dim] with 16-byte chunks XOR-swizzled within
// aligned groups of G chunks so that both read patterns of the 16x16 layout
// are free of bank conflicts on gfx950's LDS (64 banks of 4 bytes):
//   * row fragments (ds_read_b128; lane l reads chunk 4e + l/16 of row l%16):
//     the LDS serves 16 lanes per cycle, lanes 0-7 with 24-31, 8-15 with
//     16-23, 32-39 with 56-63 and 40-47 with 48-55 (measured with
//     SQ_LDS_BANK_CONFLICT on probe patterns), so rows r and r+8 of chunks
//     4e and 4e+1 (or 4e+2 and 4e+3) meet in one cycle and must take
//     different 16-byte bank groups;
//   * transposing reads (ds_read_b64_tr_b16): 32 lanes read a 32-byte chunk
//     pair of 8 consecutive rows.
// Rows of whole 256-byte bank lines (D = 256, 512; G = 16): swz(r) = 2(r&7),
// which sends rows r < 8 of chunk 4e to even bank groups and rows r >= 8 of
// chunk 4e+1 to odd ones.  Rows of an odd number of half lines (D = 576;
// G = 8), odd rows starting half a line later: swz(r) = r&6.  (Swizzles that
// are a bijection on the 16 rows of one chunk, such as 2(r&7) + ((r>>3)&1),
// put those row pairs in one bank group: each row fragment read then takes
// two LDS cycles per 16 lanes instead of one.)
#include "flash_common.h"

namespace pjx {

constexpr int kWQ = 64;   // query rows per dQ workgroup (16 per wave)
constexpr int kWK = 64;   // keys per dK/dV workgroup (16 per wave)
constexpr int kWT = 32;   // rows (keys) per streamed LDS tile

template <int D>
struct Row16 {
  static constexpr int ROWB = 2 * D;
  static constexpr int NC = D / 8;
  static constexpr bool FULL_LINES = (ROWB % 256) == 0;
  static constexpr int G = FULL_LINES ? 16 : 8;
  static constexpr int TILE_B = kWT * ROWB;
  static constexpr int NLD = kWT * NC / 256;  // 1 KiB loads per wave per tile
  static_assert(ROWB % 256 == 0 || ROWB % 256 == 128, "rows of whole or half bank lines");
  static_assert(NC % G == 0 && (kWT * NC) % 256 == 0, "tile shape");
  __device__ static int swz(int r) {
    return FULL_LINES ? ((r & 7) << 1) : (r & 6);
  }
};

// Per-lane LDS offsets of one tile layout's two read patterns.
template <typename E, int D>
struct Offs16 {
  using R = Row16<D>;
  static constexpr int PR = R::G / 4;  // period (in 32-dim steps) of row reads
  static constexpr int PT = R::G / 2;  // period (in 16-dim blocks) of transposing reads
  uint32_t row[PR];  // A = X[16 rows][32 dims]: row c, chunk 4*st + qd
  uint32_t tr[PT];   // A = X^T[16 dims][32 rows]: rows 4qd + s/4 (+16), dims 16i + 4(s%4)
  uint32_t voff[R::NLD];  // buffer->LDS sources: unit p = (NLD*w + j)*64 + lane
  __device__ void init(int lane, int w, uint32_t rowstride) {
    const int c = lane & 15, qd = lane >> 4;
#pragma unroll
    for (int e = 0; e < PR; ++e) row[e] = c * R::ROWB + 16 * ((4 * e + qd) ^ R::swz(c));
    const int rl = 4 * qd + (c >> 2), b = (c & 3) >> 1;
#pragma unroll
    for (int e = 0; e < PT; ++e) tr[e] = rl * R::ROWB + 16 * ((2 * e + b) ^ R::swz(rl)) + 8 * (c & 1);
#pragma unroll
    for (int j = 0; j < R::NLD; ++j) {
      const int p = (R::NLD * w + j) * 64 + lane, r = p / R::NC, slot = p % R::NC;
      voff[j] = r * rowstride + 16 * (slot ^ R::swz(r));
    }
  }
  // Row fragment of 32-dim step st, rows 16*rb .. +15 of the tile.
  __device__ typename E::v8 rows(const unsigned char* tile, int rb, int st) const {
    return E::as8(*(const u32x4*)(tile + 16 * rb * R::ROWB + 16 * R::G * (st / PR) + row[st % PR]));
  }
  // Transposed fragment of dims 16i .. +15 over the tile's 32 rows in k-slot
  // order (slot 8qd + j <-> row 16(j/4) + 4qd + j%4).
  __device__ typename E::v8 trans(const unsigned char* tile, int i) const {
    const unsigned char* p = tile + 16 * R::G * (i / PT) + tr[i % PT];
    const u32x2 lo = lds_read_tr16(p);
    const u32x2 hi = lds_read_tr16(p + 16 * R::ROWB);
    const u32x4 v = {lo[0], lo[1], hi[0], hi[1]};
    return E::as8(v);
  }
  // Copies rows [r0, r0 + n) (n >= 1) of a global tensor with row stride
  // `rowstride` into a tile; rows past n read as zero.
  __device__ void load(unsigned char* tile, const unsigned char* base, uint32_t rowstride, int n, int w) const {
    const uint32_t bytes = (uint32_t)(n - 1) * rowstride + R::ROWB;
    const rsrc_t rs = make_rsrc(base, bytes);
#pragma unroll
    for (int j = 0; j < R::NLD; ++j) buffer_load_lds16(rs, tile + (R::NLD * w + j) * 1024, voff[j]);
  }
};

// Two f32x4 C blocks (k slots j < 4 from a, j >= 4 from b) as a 16-bit B operand.
template <typename E>
__device__ __forceinline__ typename E::v8 pack_slots(const f32x4& a, const f32x4& b) {
  const u32x4 pk = {E::pack2(a[0], a[1]), E::pack2(a[2], a[3]), E::pack2(b[0], b[1]), E::pack2(b[2], b[3])};
  return E::as8(pk);
}

// ---------------------------------------------------------------------------
// dQ (and delta, lse*log2e): one workgroup per (64-query tile, batch, head).
// ---------------------------------------------------------------------------
template <typename E, int D, int DV, bool SHARED, int BIAS, int EXT>
__global__ __launch_bounds__(kThreads, 1) void wide_bwd_dq_kernel(WideBwdArgs ba) {
  // BIAS: 0 none, 1 dense bias, 2 dense bias and its gradient (ba.dbias)
  constexpr bool HB = BIAS != 0, DB = BIAS == 2;
  const FlashArgs& a = ba.f;
  using OK = Offs16<E, D>;
  using OV = Offs16<E, DV>;
  constexpr int KT_B = Row16<D>::TILE_B;
  constexpr int STAGE_B = SHARED ? KT_B : KT_B + Row16<DV>::TILE_B;
  constexpr int KS = D / 32, VS = DV / 32, ND = D / 16;
  static_assert(!SHARED || DV <= D, "values are a prefix of the latent row");
  __shared__ __attribute__((aligned(1024))) unsigned char smem0[STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char smem1[STAGE_B];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, qd = lane >> 4;
  const int BH = a.B * a.Hq;
  const int n_qt = (a.Lq + kWQ - 1) / kWQ;
  const int bh = (int)blockIdx.x % BH;
  const int qt = n_qt - 1 - (int)blockIdx.x / BH;  // heaviest causal tile first
  const int b = bh / a.Hq, h = bh % a.Hq, hkv = h / (a.Hq / a.Hkv);
  const int q0 = qt * kWQ;
  const int qw = __builtin_amdgcn_readfirstlane(q0 + 16 * w);
  const int qi = qw + c;
  const int q_hi = min(a.Lq, a.q_valid);
  int kv_end = min(a.Lk, a.kv_valid);
  if (a.kv_lengths) kv_end = min(kv_end, max(a.kv_lengths[b], 0));
  const bool row_in = qi < a.Lq, row_ok = qi < q_hi;
  // keys this block visits: [kv_begin, kv_stop)
  int kv_begin = 0, kv_stop = kv_end;
  if (q0 >= q_hi) {
    kv_stop = 0;
  } else if constexpr (EXT > 0) {
    int lo0, hi0, lo1, hi1;
    row_bounds(a.m, a.causal, b, kv_end, q_hi, q0, lo0, hi0);
    row_bounds(a.m, a.causal, b, kv_end, q_hi, min(q0 + kWQ, q_hi) - 1, lo1, hi1);
    kv_begin = (max(lo0, 0) / kWT) * kWT;
    kv_stop = max(min(hi1 + 1, kv_end), 0);
  } else if (a.causal) {
    kv_stop = min(kv_stop, min(q0 + kWQ, q_hi));
  }
  // this lane's key interval and the wave's (extended masks)
  int lo = 0, hi = -1, lo_first = 0, hi_last = -1, segq = 0;
  HeadMods hm = {0.f, 1.f};
  if constexpr (EXT > 0) {
    int t0, t1;
    row_bounds(a.m, a.causal, b, kv_end, q_hi, qi, lo, hi);
    row_bounds(a.m, a.causal, b, kv_end, q_hi, qw, lo_first, t0);
    row_bounds(a.m, a.causal, b, kv_end, q_hi, min(qw + 15, q_hi - 1), t1, hi_last);
    if (a.m.seg_q && row_in) segq = a.m.seg_q[(size_t)b * a.Lq + qi];
    hm = head_mods(a.m, h);
  }
  const bool wave_any_row = qw < q_hi;

  // Q^T, dO^T as B operands (lane: row qi, dims 32*st + 8*qd + [0,8)) and
  // delta = sum_d o*do over the DV output dims.
  typename E::v8 qf[KS], dof[VS];
  float dsum = 0.f;
  {
    const uint16_t* qrow = (const uint16_t*)a.q + ((size_t)(b * a.Lq + (row_in ? qi : 0)) * a.Hq + h) * D;
    const size_t ooff = ((size_t)(b * a.Lq + (row_in ? qi : 0)) * a.Hq + h) * DV;
    const uint16_t* drow = (const uint16_t*)ba.dout + ooff;
    const uint16_t* orow = (const uint16_t*)a.o + ooff;
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      u32x4 r = {0u, 0u, 0u, 0u};
      if (row_in) r = *(const u32x4*)(qrow + 32 * st + 8 * qd);
      qf[st] = E::as8(r);
    }
#pragma unroll
    for (int st = 0; st < VS; ++st) {
      u32x4 rd = {0u, 0u, 0u, 0u}, ro = rd;
      if (row_in) {
        rd = *(const u32x4*)(drow + 32 * st + 8 * qd);
        ro = *(const u32x4*)(orow + 32 * st + 8 * qd);
      }
      dof[st] = E::as8(rd);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dsum = fmaf(E::lo(ro[j]), E::lo(rd[j]), fmaf(E::hi(ro[j]), E::hi(rd[j]), dsum));
    }
  }
  const float delta = xor32_sum(xor16_sum(dsum));
  const float dsc = delta * a.scale;  // the workspace holds delta * sm_scale
  float lse2 = 0.f;
  const size_t lidx = ((size_t)b * a.Hq + h) * a.Lq + qi;
  if (row_in) {
    lse2 = a.lse[lidx] * kLog2e;
    if (qd == 0) {
      ba.delta[lidx] = dsc;
      ba.lse2[lidx] = lse2;
    }
  }
  const float* brow = nullptr;
  if constexpr (HB)
    brow = a.bias + (size_t)b * a.bias_bstride + (size_t)h * a.bias_hstride + (size_t)(row_in ? qi : 0) * a.Lk;
  const float cx = (HB || EXT == 2) ? kLog2e : a.scale * kLog2e;
  const uint32_t rowstride = (uint32_t)a.Hkv * 2 * D;  // K / V rows (Hkv heads of D dims)
  const uint32_t vrowstride = (uint32_t)a.Hkv * 2 * DV;
  const unsigned char* Kb = (const unsigned char*)a.k + ((size_t)b * a.Lk * a.Hkv + hkv) * (2 * D);
  const unsigned char* Vb = (const unsigned char*)a.v + ((size_t)b * a.Lk * a.Hkv + hkv) * (2 * DV);

  OK ok;
  ok.init(lane, w, rowstride);
  OV ov;
  if constexpr (!SHARED) ov.init(lane, w, vrowstride);

  f32x4 acc[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) acc[i] = f32x4{};

  const int t_begin = kv_begin / kWT;
  const int n_tiles = max((kv_stop + kWT - 1) / kWT - t_begin, 0);

  auto issue = [&](int t, unsigned char* st) {
    const int k0 = (t_begin + t) * kWT;
    const int n = min(kWT, kv_stop - k0);
    ok.load(st, Kb + (size_t)k0 * rowstride, rowstride, n, w);
    if constexpr (!SHARED) ov.load(st + KT_B, Vb + (size_t)k0 * vrowstride, vrowstride, n, w);
  };

  auto compute = [&](int t, const unsigned char* ks) {
    const int k0 = (t_begin + t) * kWT;
    if constexpr (EXT > 0) {
      if (!wave_any_row || k0 > hi_last || k0 + kWT - 1 < lo_first) return;
    } else {
      if (!wave_any_row || (a.causal && k0 > qw + 15)) return;
    }
    const unsigned char* vs = ks + KT_B;
    // s[kb][r] = S^T[key k0 + 16kb + 4qd + r][row qi]; dp likewise.
    f32x4 s[2], dp[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f32x4{};
      dp[kb] = f32x4{};
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        const typename E::v8 kf = ok.rows(ks, kb, st);
        s[kb] = E::mma16(kf, qf[st], s[kb]);
        if constexpr (SHARED) {
          if (st < VS) dp[kb] = E::mma16(kf, dof[st], dp[kb]);
        }
      }
      if constexpr (!SHARED) {
#pragma unroll
        for (int st = 0; st < VS; ++st) dp[kb] = E::mma16(ov.rows(vs, kb, st), dof[st], dp[kb]);
      }
    }
    {
      // Each row fragment read 6 reads ahead of its MFMAs.  Reads in program
      // order: per kb, KS K rows (each feeding S, and dP for st < VS with the
      // shared latent), then VS V rows.
      constexpr int NR = 2 * (KS + (SHARED ? 0 : VS));
      __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
      for (int i_ = 0; i_ < NR; ++i_) {
        const int st_ = i_ % (NR / 2);
        if (SHARED && st_ < VS)
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        else
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i_ + 6 < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    f32x4 dbv[2];
    const int kbase = k0 + 4 * qd;
    if constexpr (EXT == 2) {
      const bool soft = a.m.softcap > 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int kk = kbase + 16 * kb;
        f32x4 bv = {0.f, 0.f, 0.f, 0.f};
        if constexpr (HB) {
          if (row_in) bv = ((a.Lk & 3) == 0) ? load_bias4<true>(brow, kk, a.Lk) : load_bias4<false>(brow, kk, a.Lk);
        }
        int4 sg = {0, 0, 0, 0};
        if (a.m.seg_k) sg = seg4(a.m.seg_k, b, kk, a.Lk);
        const int sgv[4] = {sg.x, sg.y, sg.z, sg.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kj = kk + r;
          float gg;
          const float raw = s[kb][r] * a.scale;
          const float x = soft ? modify_score<true>(a.m, hm, raw, bv[r], qi, kj, gg)
                               : modify_score<false>(a.m, hm, raw, bv[r], qi, kj, gg);
          const bool keep = kj >= lo && kj <= hi &&
                            (!a.m.seg_q || (a.m.seg_lt ? kj < segq : sgv[r] == segq));
          const float p = keep ? fast_exp2(fmaf(x, cx, -lse2)) : 0.f;
          const float tt = p * (dp[kb][r] - delta);
          if constexpr (DB) dbv[kb][r] = tt;
          s[kb][r] = tt * a.scale * gg;
        }
      }
    } else {
      if constexpr (HB) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const int kk = kbase + 16 * kb;
          f32x4 bv = {0.f, 0.f, 0.f, 0.f};
          if (row_in) bv = ((a.Lk & 3) == 0) ? load_bias4<true>(brow, kk, a.Lk) : load_bias4<false>(brow, kk, a.Lk);
#pragma unroll
          for (int r = 0; r < 4; ++r) s[kb][r] = fmaf(s[kb][r], a.scale, bv[r]);
        }
      }
      const bool need_mask = (k0 + kWT > kv_end) || (a.causal && k0 + kWT - 1 > qw) || (qw + 15 >= q_hi);
      if (need_mask) {
        int lim = kv_end - 1 - kbase;
        if (a.causal) lim = min(lim, qi - kbase);
        if (!row_ok) lim = -1;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (16 * kb + r > lim) s[kb][r] = -INFINITY;
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = fast_exp2(fmaf(s[kb][r], cx, -lse2));
          if constexpr (DB) {
            const float tt = p * (dp[kb][r] - delta);
            dbv[kb][r] = tt;
            s[kb][r] = tt * a.scale;
          } else {
            s[kb][r] = p * fmaf(dp[kb][r], a.scale, -dsc);  // p (dp - delta) scale
          }
        }
    }
    if constexpr (DB) {
      if (row_in) {
        float* row = ba.dbias + (((size_t)b * a.Hq + h) * a.Lq + qi) * a.Lk;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const int kk = kbase + 16 * kb;
          if ((a.Lk & 3) == 0 && kk + 3 < a.Lk) {
            *(f32x4*)(row + kk) = dbv[kb];
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (kk + r < a.Lk) row[kk + r] = dbv[kb][r];
          }
        }
      }
    }
    // dQ^T[16i + 4qd + r][row] += K^T dS^T
    const typename E::v8 dsb = pack_slots<E>(s[0], s[1]);
#pragma unroll
    for (int i = 0; i < ND; ++i) acc[i] = E::mma16(ok.trans(ks, i), dsb, acc[i]);
    PJX_SCHED_LDS_READS_AHEAD(ND, 6, 2);  // transposed K fragments 6 MFMAs ahead
  };

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

  if (row_in) {
    uint16_t* drow = (uint16_t*)ba.dq + ((size_t)(b * a.Lq + qi) * a.Hq + h) * D;
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      u32x2 pk;
      pk[0] = E::pack2(acc[i][0], acc[i][1]);
      pk[1] = E::pack2(acc[i][2], acc[i][3]);
      *(u32x2*)(drow + 16 * i + 4 * qd) = pk;
    }
  }
}

// ---------------------------------------------------------------------------
// dK, dV (or dC = dK + dV of the shared latent): one workgroup per (64-key
// tile, batch, KV head, query-head group).
// ---------------------------------------------------------------------------
template <typename E, int D, int DV, bool SHARED, bool BIAS, int EXT>
__global__ __launch_bounds__(kThreads, 1) void wide_bwd_dkdv_kernel(WideBwdArgs ba) {
  const FlashArgs& a = ba.f;
  using OQ = Offs16<E, D>;
  using OD = Offs16<E, DV>;
  constexpr int QT_B = Row16<D>::TILE_B, DT_B = Row16<DV>::TILE_B;
  // lse*log2e and delta * sm_scale of the tile's rows, one 64-float slot each (the
  // 4-byte buffer->LDS load writes one float per lane; lanes 32..63 fill the
  // unused upper half)
  constexpr int SMALL_B = 2 * 64 * 4;
  constexpr int STAGE_B = QT_B + DT_B + SMALL_B;
  constexpr int KS = D / 32, VS = DV / 32, ND = D / 16, NV = DV / 16;
  static_assert(!SHARED || DV <= D, "values are a prefix of the latent row");
  __shared__ __attribute__((aligned(1024))) unsigned char smem0[STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char smem1[STAGE_B];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, qd = lane >> 4;
  const int nsplit = ba.nsplit;
  const int split = (int)blockIdx.x % nsplit;
  const int rest = (int)blockIdx.x / nsplit;
  const int BH = a.B * a.Hkv;
  const int bh = rest % BH;
  const int k0 = (rest / BH) * kWK;
  const int b = bh / a.Hkv, hkv = bh % a.Hkv;
  const int G = a.Hq / a.Hkv;
  const int gs = G / nsplit;              // query heads of this group
  const int h_first = hkv * G + split * gs;
  const int kw = __builtin_amdgcn_readfirstlane(k0 + 16 * w);
  const int key = kw + c;
  int kv_end = min(a.Lk, a.kv_valid);
  if (a.kv_lengths) kv_end = min(kv_end, max(a.kv_lengths[b], 0));
  const int q_hi = min(a.Lq, a.q_valid);
  // query rows that can see a key of this tile: [q_begin, q_end)
  int q_begin = a.causal ? (k0 / kWT) * kWT : 0;
  int q_end = q_hi;
  int qlo = 0, qhi = q_hi - 1, wq_first = 0, wq_last = q_hi - 1, segk = 0;
  if constexpr (EXT > 0) {
    q_end = q_begin = 0;
    if (k0 < kv_end) {
      int a0, a1, b0, b1;
      key_bounds(a.m, a.causal, b, kv_end, q_hi, k0, a0, a1);
      key_bounds(a.m, a.causal, b, kv_end, q_hi, min(k0 + kWK, kv_end) - 1, b0, b1);
      q_begin = (max(a0, 0) / kWT) * kWT;
      q_end = b1 + 1;
    }
    key_bounds(a.m, a.causal, b, kv_end, q_hi, key, qlo, qhi);
    if (kw < kv_end) {
      int t0, t1;
      key_bounds(a.m, a.causal, b, kv_end, q_hi, kw, wq_first, t0);
      key_bounds(a.m, a.causal, b, kv_end, q_hi, min(kw + 16, kv_end) - 1, t1, wq_last);
    }
    if (a.m.seg_k && key < a.Lk) segk = a.m.seg_k[(size_t)b * a.Lk + key];
  }
  const int n_qt = (k0 < kv_end && q_end > q_begin) ? (q_end - q_begin + kWT - 1) / kWT : 0;
  const int n_tiles = gs * n_qt;

  // K^T (and V^T) as B operands: lane holds key `key`, dims 32*st + 8*qd + [0,8).
  typename E::v8 kf[KS], vf[SHARED ? 1 : VS];
  {
    const bool kin = key < a.Lk;
    const uint16_t* krow = (const uint16_t*)a.k + ((size_t)(b * a.Lk + (kin ? key : 0)) * a.Hkv + hkv) * D;
    const uint16_t* vrow = (const uint16_t*)a.v + ((size_t)(b * a.Lk + (kin ? key : 0)) * a.Hkv + hkv) * DV;
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      u32x4 r = {0u, 0u, 0u, 0u};
      if (kin) r = *(const u32x4*)(krow + 32 * st + 8 * qd);
      kf[st] = E::as8(r);
    }
    if constexpr (!SHARED) {
#pragma unroll
      for (int st = 0; st < VS; ++st) {
        u32x4 r = {0u, 0u, 0u, 0u};
        if (kin) r = *(const u32x4*)(vrow + 32 * st + 8 * qd);
        vf[st] = E::as8(r);
      }
    }
  }
  const float cx = (BIAS || EXT == 2) ? kLog2e : a.scale * kLog2e;
  const uint32_t qrowstride = (uint32_t)a.Hq * 2 * D;
  const uint32_t drowstride = (uint32_t)a.Hq * 2 * DV;
  OQ oq;
  oq.init(lane, w, qrowstride);
  OD od;
  od.init(lane, w, drowstride);

  f32x4 acck[ND], accv[SHARED ? 1 : NV];
#pragma unroll
  for (int i = 0; i < ND; ++i) acck[i] = f32x4{};
  if constexpr (!SHARED) {
#pragma unroll
    for (int i = 0; i < NV; ++i) accv[i] = f32x4{};
  }

  // Query tiles last to first, the group's heads innermost: the workgroups of
  // one head group's key tiles (same XCD, running together) then stream the
  // same Q / dO tile at the same time, so all but the first read it from L2.
  auto tile_head = [&](int t) { return h_first + t % gs; };
  auto tile_q0 = [&](int t) { return q_begin + (n_qt - 1 - t / gs) * kWT; };

  auto issue = [&](int t, unsigned char* st) {
    const int h = tile_head(t), q0 = tile_q0(t);
    const int n = max(min(kWT, a.Lq - q0), 1);
    oq.load(st, (const unsigned char*)a.q + ((size_t)(b * a.Lq + q0) * a.Hq + h) * (2 * D), qrowstride, n, w);
    od.load(st + QT_B, (const unsigned char*)ba.dout + ((size_t)(b * a.Lq + q0) * a.Hq + h) * (2 * DV),
            drowstride, n, w);
    if (w < 2) {
      const size_t loff = ((size_t)b * a.Hq + h) * a.Lq + q0;
      const rsrc_t rl = make_rsrc((w == 0 ? ba.lse2 : ba.delta) + loff, (uint32_t)n * 4);
      buffer_load_lds4(rl, st + QT_B + DT_B + w * 256, 4 * (lane & 31));
    }
  };

  auto compute = [&](int t, const unsigned char* st) {
    const int h = tile_head(t), q0 = tile_q0(t);
    if (kw >= kv_end || q0 >= q_hi) return;
    if constexpr (EXT > 0) {
      if (q0 > wq_last || q0 + kWT - 1 < wq_first) return;
    } else {
      if (a.causal && q0 + kWT - 1 < kw) return;  // every row before the wave's first key
    }
    const unsigned char* qs = st;
    const unsigned char* dos = st + QT_B;
    const float* lsm = (const float*)(st + QT_B + DT_B);
    const float* dlm = lsm + 64;
    // sx[rb][r] = S[row q0 + 16rb + 4qd + r][key]; dpx likewise.
    f32x4 sx[2], dpx[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      sx[rb] = f32x4{};
      dpx[rb] = f32x4{};
#pragma unroll
      for (int s = 0; s < KS; ++s) sx[rb] = E::mma16(oq.rows(qs, rb, s), kf[s], sx[rb]);
#pragma unroll
      for (int s = 0; s < VS; ++s)
        dpx[rb] = E::mma16(od.rows(dos, rb, s), SHARED ? kf[s] : vf[s], dpx[rb]);
    }
    const float* bbase = nullptr;
    if constexpr (BIAS) bbase = a.bias + (size_t)b * a.bias_bstride + (size_t)h * a.bias_hstride;
    HeadMods hm = {0.f, 1.f};
    if constexpr (EXT == 2) hm = head_mods(a.m, h);
    const bool soft = EXT == 2 && a.m.softcap > 0.f;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int q4 = q0 + 16 * rb + 4 * qd;
      const f32x4 l4 = *(const f32x4*)(lsm + 16 * rb + 4 * qd);
      const f32x4 d4 = *(const f32x4*)(dlm + 16 * rb + 4 * qd);
      int4 sg = {0, 0, 0, 0};
      if (EXT == 2 && a.m.seg_q) sg = seg4(a.m.seg_q, b, q4, a.Lq);
      const int sgv[4] = {sg.x, sg.y, sg.z, sg.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qr = q4 + r;
        float bv = 0.f;
        if constexpr (BIAS) bv = (qr < a.Lq && key < a.Lk) ? bbase[(size_t)qr * a.Lk + key] : 0.f;
        float x, gg = 1.f;
        bool keep;
        if constexpr (EXT == 2) {
          const float raw = sx[rb][r] * a.scale;
          x = soft ? modify_score<true>(a.m, hm, raw, bv, qr, key, gg) : modify_score<false>(a.m, hm, raw, bv, qr, key, gg);
          keep = qr >= qlo && qr <= qhi && (!a.m.seg_q || (a.m.seg_lt ? key < sgv[r] : sgv[r] == segk));
        } else {
          x = BIAS ? fmaf(sx[rb][r], a.scale, bv) : sx[rb][r];
          keep = key < kv_end && qr < q_hi && (!a.causal || qr >= key);
        }
        const float p = keep ? fast_exp2(fmaf(x, cx, -l4[r])) : 0.f;
        sx[rb][r] = p;
        dpx[rb][r] = p * fmaf(dpx[rb][r], a.scale, -d4[r]) * gg;
      }
    }
    const typename E::v8 pb = pack_slots<E>(sx[0], sx[1]);
    const typename E::v8 dsb = pack_slots<E>(dpx[0], dpx[1]);
    // dK^T[16i + 4qd + r][key] += Q^T dS;  dV^T += dO^T P (into dK^T with the latent)
#pragma unroll
    for (int i = 0; i < ND; ++i) acck[i] = E::mma16(oq.trans(qs, i), dsb, acck[i]);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if constexpr (SHARED)
        acck[i] = E::mma16(od.trans(dos, i), pb, acck[i]);
      else
        accv[i] = E::mma16(od.trans(dos, i), pb, accv[i]);
    }
  };

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

  if (key >= a.Lk) return;
  const size_t krow = (size_t)(b * a.Lk + key) * a.Hkv + hkv;
  if (nsplit == 1) {
    uint16_t* dkrow = (uint16_t*)ba.dk + krow * D;
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      const u32x2 pk = {E::pack2(acck[i][0], acck[i][1]), E::pack2(acck[i][2], acck[i][3])};
      *(u32x2*)(dkrow + 16 * i + 4 * qd) = pk;
    }
    if constexpr (!SHARED) {
      uint16_t* dvrow = (uint16_t*)ba.dv + krow * DV;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const u32x2 pv = {E::pack2(accv[i][0], accv[i][1]), E::pack2(accv[i][2], accv[i][3])};
        *(u32x2*)(dvrow + 16 * i + 4 * qd) = pv;
      }
    }
  } else {
    // fp32 partial of this head group: [split][B*Lk*Hkv][D] then (separate
    // K / V) [split][B*Lk*Hkv][DV] after all K partials.
    const size_t nrows = (size_t)a.B * a.Lk * a.Hkv;
    float* pk = ba.part + ((size_t)split * nrows + krow) * D;
#pragma unroll
    for (int i = 0; i < ND; ++i) *(f32x4*)(pk + 16 * i + 4 * qd) = acck[i];
    if constexpr (!SHARED) {
      float* pv = ba.part + (size_t)nsplit * nrows * D + ((size_t)split * nrows + krow) * DV;
#pragma unroll
      for (int i = 0; i < NV; ++i) *(f32x4*)(pv + 16 * i + 4 * qd) = accv[i];
    }
  }
}

// ---------------------------------------------------------------------------
// dK and dV (or dC = dK + dV of the shared latent) without bias or extended
// masks: the workgroup of wide_bwd_dkdv_kernel (64 keys, one query-head group,
// Q / dO tiles of 32 rows through LDS) with the gradient update split by
// columns instead of keys.  Wave w forms S, dP, P and dS for keys
// k0 + 16w .. +15 as there, and posts P and dS (its two 16-bit B operands,
// 1 KiB each) to LDS.  After a barrier it accumulates, for the 16-column
// blocks i = w + 4j over all 64 keys, dK^T += Q^T dS and (blocks below DV/16)
// dV^T += dO^T P; with the shared latent both go into one accumulator.  A
// wave then reads the transposed Q / dO fragments of its own blocks only (a
// quarter of the tile) where the key split reads all of them in every wave.
// ---------------------------------------------------------------------------
// At D = 256 (separate K / V) two workgroups share a CU: 73 KiB of LDS each,
// and the instance fits 256 registers without spills (250 VGPRs).  The latent
// widths need 147 KiB of LDS and run one.
// DS (the dS route): each compute() also stores the wave's rounded dS block
// (16 keys x 32 queries, zeros where no row of the tile sees the wave's keys)
// into ba.ds; see wide_bwd_dq_ds_kernel for the layout.
template <typename E, int D, int DV, bool SHARED, bool DS>
__device__ __forceinline__ void wide_dc_body(const WideBwdArgs& ba) {
  const FlashArgs& a = ba.f;
  using RQ = Row16<D>;
  using RD = Row16<DV>;
  using OQ = Offs16<E, D>;
  using OD = Offs16<E, DV>;
  constexpr int QT_B = RQ::TILE_B, DT_B = RD::TILE_B;
  constexpr int SMALL_B = 2 * 64 * 4;  // lse*log2e and delta * sm_scale of the tile's rows
  constexpr int STAGE_B = QT_B + DT_B + SMALL_B;
  constexpr int KS = D / 32, VS = DV / 32, ND = D / 16, NV = DV / 16;
  constexpr int NJ = ND / 4, NJV = NV / 4;  // column blocks per wave, those with dV first
  static_assert(ND % 4 == 0 && NV % 4 == 0 && DV <= D, "column blocks split evenly over the 4 waves");
  static_assert(SHARED || DV == D, "separate K / V of one width");
  __shared__ __attribute__((aligned(1024))) unsigned char smem0[STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char smem1[STAGE_B];
  __shared__ __attribute__((aligned(1024))) u32x4 xp[4 * 2 * 64];  // [wave][P, dS][lane]

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, qd = lane >> 4;
  const int nsplit = ba.nsplit;
  const int split = (int)blockIdx.x % nsplit;
  const int rest = (int)blockIdx.x / nsplit;
  const int BH = a.B * a.Hkv;
  const int bh = rest % BH;
  const int k0 = (rest / BH) * kWK;
  const int b = bh / a.Hkv, hkv = bh % a.Hkv;
  const int G = a.Hq / a.Hkv;
  const int gs = G / nsplit;  // query heads of this group
  const int h_first = hkv * G + split * gs;
  const int kw = __builtin_amdgcn_readfirstlane(k0 + 16 * w);
  const int key = kw + c;
  int kv_end = min(a.Lk, a.kv_valid);
  if (a.kv_lengths) kv_end = min(kv_end, max(a.kv_lengths[b], 0));
  const int q_hi = min(a.Lq, a.q_valid);
  const int q_begin = a.causal ? (k0 / kWT) * kWT : 0;
  const int n_qt = (k0 < kv_end && q_hi > q_begin) ? (q_hi - q_begin + kWT - 1) / kWT : 0;
  const int n_tiles = gs * n_qt;

  // K^T (and V^T) as the B operands of S and dP: lane holds key `key`, dims
  // 32*st + 8*qd + [0,8).
  typename E::v8 kf[KS], vf[SHARED ? 1 : VS];
  {
    const bool kin = key < a.Lk;
    const size_t kr = (size_t)(b * a.Lk + (kin ? key : 0)) * a.Hkv + hkv;
    const uint16_t* krow = (const uint16_t*)a.k + kr * D;
    const uint16_t* vrow = (const uint16_t*)a.v + kr * DV;
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      u32x4 r = {0u, 0u, 0u, 0u};
      if (kin) r = *(const u32x4*)(krow + 32 * st + 8 * qd);
      kf[st] = E::as8(r);
    }
    if constexpr (!SHARED) {
#pragma unroll
      for (int st = 0; st < VS; ++st) {
        u32x4 r = {0u, 0u, 0u, 0u};
        if (kin) r = *(const u32x4*)(vrow + 32 * st + 8 * qd);
        vf[st] = E::as8(r);
      }
    }
  }
  const float cx = a.scale * kLog2e;
  const uint32_t qrowstride = (uint32_t)a.Hq * 2 * D;
  const uint32_t drowstride = (uint32_t)a.Hq * 2 * DV;
  OQ oq;
  oq.init(lane, w, qrowstride);
  OD od;
  od.init(lane, w, drowstride);
  // Transposed-read offsets (Offs16::trans) of this wave's column blocks w + 4j.
  uint32_t offq[NJ], offd[NJV];
  {
    const int rl = 4 * qd + (c >> 2), bsel = (c & 3) >> 1;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int i = w + 4 * j;
      offq[j] = 16 * RQ::G * (i / OQ::PT) + rl * RQ::ROWB + 16 * ((2 * (i % OQ::PT) + bsel) ^ RQ::swz(rl)) + 8 * (c & 1);
    }
#pragma unroll
    for (int j = 0; j < NJV; ++j) {
      const int i = w + 4 * j;
      offd[j] = 16 * RD::G * (i / OD::PT) + rl * RD::ROWB + 16 * ((2 * (i % OD::PT) + bsel) ^ RD::swz(rl)) + 8 * (c & 1);
    }
  }
  auto trans_at = [](const unsigned char* tile, uint32_t off, int rowb) {
    const u32x2 lo = lds_read_tr16(tile + off);
    const u32x2 hi = lds_read_tr16(tile + off + 16 * rowb);
    const u32x4 v = {lo[0], lo[1], hi[0], hi[1]};
    return E::as8(v);
  };

  // acc[j][kb][r] = dK^T (dC^T) [16 (w + 4j) + 4qd + r][k0 + 16kb + c]; accv likewise dV^T
  f32x4 acc[NJ][4], accv[SHARED ? 1 : NJV][4];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) acc[j][kb] = f32x4{};
  if constexpr (!SHARED) {
#pragma unroll
    for (int j = 0; j < NJV; ++j)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) accv[j][kb] = f32x4{};
  }

  // Query tiles last to first, the group's heads innermost (as in wide_bwd_dkdv_kernel).
  auto tile_head = [&](int t) { return h_first + t % gs; };
  auto tile_q0 = [&](int t) { return q_begin + (n_qt - 1 - t / gs) * kWT; };

  auto issue = [&](int t, unsigned char* st) {
    const int h = tile_head(t), q0 = tile_q0(t);
    const int n = max(min(kWT, a.Lq - q0), 1);
    oq.load(st, (const unsigned char*)a.q + ((size_t)(b * a.Lq + q0) * a.Hq + h) * (2 * D), qrowstride, n, w);
    od.load(st + QT_B, (const unsigned char*)ba.dout + ((size_t)(b * a.Lq + q0) * a.Hq + h) * (2 * DV),
            drowstride, n, w);
    if (w < 2) {
      const size_t loff = ((size_t)b * a.Hq + h) * a.Lq + q0;
      const rsrc_t rl = make_rsrc((w == 0 ? ba.lse2 : ba.delta) + loff, (uint32_t)n * 4);
      buffer_load_lds4(rl, st + QT_B + DT_B + w * 256, 4 * (lane & 31));
    }
  };

  // DS: element offset of this wave's dS block for the next tile, advanced
  // per tile in the tile order (heads innermost, query tiles last to first)
  // with uniform adds; computing it from t (t % gs, t / gs by the runtime
  // group size) put a division on the vector unit into the tile's block and
  // broke the S / dP fragment read-ahead order of the latent instance.
  const long ds_plane = (long)ba.ds_nq32 * ba.ds_nk16 * 512;  // one query head's blocks
  const long ds_wrap = -((long)(gs - 1) * ds_plane + (long)(kWT / 32) * ba.ds_nk16 * 512);
  long ds_off = 0;
  int ds_hh = 0;  // head of the next tile within the group
  if constexpr (DS)
    ds_off = (((long)(b * a.Hq + h_first) * ba.ds_nq32 + (q_begin + (n_qt - 1) * kWT) / 32) * ba.ds_nk16 + kw / 16) * 512;

  auto compute = [&](int t, const unsigned char* st) {
    const int q0 = tile_q0(t);
    long my_ds = 0;
    if constexpr (DS) {
      my_ds = ds_off;
      const bool wrap = ds_hh + 1 == gs;  // next tile: the group's first head, one query tile lower
      ds_hh = wrap ? 0 : ds_hh + 1;
      ds_off += wrap ? ds_wrap : ds_plane;
    }
    // uniform over the workgroup; never taken for t < n_tiles (tile_q0 < q_hi),
    // which the DS ring's store count relies on
    if (q0 >= q_hi) return;
    const unsigned char* qs = st;
    const unsigned char* dos = st + QT_B;
    // P and dS of this wave's keys (zero where no row of the tile sees them)
    u32x4 pbv = {0u, 0u, 0u, 0u}, dsv = pbv;
    if (kw < kv_end && !(a.causal && q0 + kWT - 1 < kw)) {
      const float* lsm = (const float*)(st + QT_B + DT_B);
      const float* dlm = lsm + 64;
      f32x4 sx[2], dpx[2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        sx[rb] = f32x4{};
        dpx[rb] = f32x4{};
#pragma unroll
        for (int s = 0; s < KS; ++s) sx[rb] = E::mma16(oq.rows(qs, rb, s), kf[s], sx[rb]);
#pragma unroll
        for (int s = 0; s < VS; ++s)
          dpx[rb] = E::mma16(od.rows(dos, rb, s), SHARED ? kf[s] : vf[s], dpx[rb]);
      }
      // Each MFMA's row fragment is read from LDS 6 MFMAs ahead (at one wave
      // per SIMD the scheduler's own order waited for each read right before
      // its MFMA).
      PJX_SCHED_LDS_READS_AHEAD(2 * (KS + VS), 6, 1);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const int q4 = q0 + 16 * rb + 4 * qd;
        const f32x4 l4 = *(const f32x4*)(lsm + 16 * rb + 4 * qd);
        const f32x4 d4 = *(const f32x4*)(dlm + 16 * rb + 4 * qd);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qr = q4 + r;
          const bool keep = key < kv_end && qr < q_hi && (!a.causal || qr >= key);
          const float p = keep ? fast_exp2(fmaf(sx[rb][r], cx, -l4[r])) : 0.f;
          sx[rb][r] = p;
          dpx[rb][r] = p * fmaf(dpx[rb][r], a.scale, -d4[r]);
        }
      }
      pbv = __builtin_bit_cast(u32x4, pack_slots<E>(sx[0], sx[1]));
      dsv = __builtin_bit_cast(u32x4, pack_slots<E>(dpx[0], dpx[1]));
    }
    xp[(2 * w) * 64 + lane] = pbv;
    xp[(2 * w + 1) * 64 + lane] = dsv;
    stage_barrier();
    if constexpr (DS) {
      // block (query block q0 / 32, key block kw / 16) of head tile_head(t):
      // lane (c, qd) holds key kw + c, queries q0 + 4qd + [0,4) then
      // q0 + 16 + 4qd + [0,4) (pack_slots), stored as 16 bytes at 16 * lane
      __builtin_nontemporal_store(dsv, (u32x4*)(ba.ds + my_ds + 8 * lane));  // read once, by the dQ kernel
    }
    typename E::v8 pk[4], dk[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      pk[kb] = E::as8(xp[(2 * kb) * 64 + lane]);
      dk[kb] = E::as8(xp[(2 * kb + 1) * 64 + lane]);
    }
    // block w + 4j: dK^T += Q^T dS, dV^T += dO^T P (below DV; into dK^T with the latent)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const typename E::v8 fq = trans_at(qs, offq[j], RQ::ROWB);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) acc[j][kb] = E::mma16(fq, dk[kb], acc[j][kb]);
      if (j < NJV) {
        const typename E::v8 fd = trans_at(dos, offd[j < NJV ? j : 0], RD::ROWB);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          if constexpr (SHARED)
            acc[j][kb] = E::mma16(fd, pk[kb], acc[j][kb]);
          else
            accv[j < NJV ? j : 0][kb] = E::mma16(fd, pk[kb], accv[j < NJV ? j : 0][kb]);
        }
      }
    }
    // The 8 exchanged P / dS fragments and the first 3 blocks' transposed
    // fragments first, then each block's 4 MFMAs followed by the reads of the
    // block 3 ahead.
    __builtin_amdgcn_sched_group_barrier(0x100, 8 + 2 * 3, 0);
#pragma unroll
    for (int g_ = 0; g_ < NJ + NJV - 3; ++g_) {
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4 * 3, 0);
  };

  // The ring of wide_bwd_dkdv_kernel; each compute adds one barrier between
  // the xp writes and reads, and the next xp writes follow the next ring
  // barrier.  With DS the ring barrier waits for this wave's tile loads only:
  // the one dS store of the last compute() (issued after them; vmcnt counts
  // in issue order) stays in flight, and the barrier is stage_barrier(), as
  // __syncthreads()'s release fence would wait for it.  Tile 0's loads are
  // waited for before the loop, so every ring wait is the same vmcnt(1) (a
  // wait that depended on a per-iteration store count made the compiler
  // duplicate the loop body: ~10x the code, and the latent instance ran at
  // half speed).  The scheduling barriers keep the store after the loads
  // issued before it.
  auto ring_wait = [&]() {
    if constexpr (DS) {
      wait_vmcnt<1>();
      stage_barrier();
    } else {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  };
  if (n_tiles > 0) issue(0, smem0);
  if constexpr (DS) wait_vmcnt<0>();
  for (int t = 0; t < n_tiles; t += 2) {
    ring_wait();
    if (t + 1 < n_tiles) issue(t + 1, smem1);
    if constexpr (DS) __builtin_amdgcn_sched_barrier(0);
    compute(t, smem0);
    if (t + 1 >= n_tiles) break;
    ring_wait();
    if (t + 2 < n_tiles) issue(t + 2, smem0);
    if constexpr (DS) __builtin_amdgcn_sched_barrier(0);
    compute(t + 1, smem1);
  }

  // Outputs as wide_bwd_dkdv_kernel's: 16-bit rows with one group, else fp32
  // partials [split][B*Lk*Hkv][D] (then, separate K / V, [split][..][DV]).
  const size_t nrows = (size_t)a.B * a.Lk * a.Hkv;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int kk = k0 + 16 * kb + c;
    if (kk >= a.Lk) continue;
    const size_t krow = (size_t)(b * a.Lk + kk) * a.Hkv + hkv;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = 16 * (w + 4 * j) + 4 * qd;
      if (nsplit == 1) {
        const u32x2 pkd = {E::pack2(acc[j][kb][0], acc[j][kb][1]), E::pack2(acc[j][kb][2], acc[j][kb][3])};
        *(u32x2*)((uint16_t*)ba.dk + krow * D + col) = pkd;
      } else {
        *(f32x4*)(ba.part + ((size_t)split * nrows + krow) * D + col) = acc[j][kb];
      }
    }
    if constexpr (!SHARED) {
#pragma unroll
      for (int j = 0; j < NJV; ++j) {
        const int col = 16 * (w + 4 * j) + 4 * qd;
        if (nsplit == 1) {
          const u32x2 pv = {E::pack2(accv[j][kb][0], accv[j][kb][1]), E::pack2(accv[j][kb][2], accv[j][kb][3])};
          *(u32x2*)((uint16_t*)ba.dv + krow * DV + col) = pv;
        } else {
          *(f32x4*)(ba.part + (size_t)nsplit * nrows * D + ((size_t)split * nrows + krow) * DV + col) = accv[j][kb];
        }
      }
    }
  }
}

template <typename E, int D, int DV, bool SHARED>
__global__ __launch_bounds__(kThreads, (D == 256 ? 2 : 1)) void wide_bwd_dc_kernel(WideBwdArgs ba) {
  wide_dc_body<E, D, DV, SHARED, false>(ba);
}

// ---------------------------------------------------------------------------
// The dS route (head dim 256, 16-bit, no bias, no extended masks; the
// caller's workspace holds the dS blocks).  At D = 256 the dQ kernel's
// recomputation of S and dP (two products of 256 dims per score) costs more
// than writing and reading back the rounded dS (2 bytes per score, whatever
// the width), so the route runs: wide_bwd_delta_kernel; wide_bwd_dc_ds_kernel,
// which also stores dS; then wide_bwd_dq_ds_kernel, one product per score.
// dS moves with non-temporal stores and loads (written once, read once; the
// key-side kernel's Q / dO rows keep the L2): C2WB -4.5% against plain ones.
// Same roundings, sums and summation order as the two-kernel route, so the
// results are bitwise those of that route.
// ---------------------------------------------------------------------------

template <typename E, int D, int DV, bool SHARED>
__global__ __launch_bounds__(kThreads, (D == 256 ? 2 : 1)) void wide_bwd_dc_ds_kernel(WideBwdArgs ba) {
  wide_dc_body<E, D, DV, SHARED, true>(ba);
}

// delta * sm_scale and lse * log2e of every query row (what wide_bwd_dq_kernel
// writes): four lanes per row, lane qd summing dims 32st + 8qd + [0,8) over
// the DV output dims in that kernel's order, then (qd 0 + qd 1) + (qd 2 + qd 3).
template <typename E, int DV>
__global__ __launch_bounds__(kThreads) void wide_bwd_delta_kernel(WideBwdArgs ba) {
  const FlashArgs& a = ba.f;
  constexpr int VS = DV / 32;
  const long rows = (long)a.B * a.Lq * a.Hq;
  const long row = (long)blockIdx.x * (kThreads / 4) + (threadIdx.x >> 2);
  const int qd = threadIdx.x & 3;
  float dsum = 0.f;
  if (row < rows) {
    const uint16_t* orow = (const uint16_t*)a.o + row * DV;
    const uint16_t* drow = (const uint16_t*)ba.dout + row * DV;
#pragma unroll
    for (int st = 0; st < VS; ++st) {
      const u32x4 ro = *(const u32x4*)(orow + 32 * st + 8 * qd);
      const u32x4 rd = *(const u32x4*)(drow + 32 * st + 8 * qd);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dsum = fmaf(E::lo(ro[j]), E::lo(rd[j]), fmaf(E::hi(ro[j]), E::hi(rd[j]), dsum));
    }
  }
  const float pair = dsum + __shfl_xor(dsum, 1);
  const float delta = pair + __shfl_xor(pair, 2);
  if (row < rows && qd == 0) {
    const int h = (int)(row % a.Hq);
    const long bq = row / a.Hq;
    const int qi = (int)(bq % a.Lq), b = (int)(bq / a.Lq);
    const size_t lidx = ((size_t)b * a.Hq + h) * a.Lq + qi;
    ba.delta[lidx] = delta * a.scale;
    ba.lse2[lidx] = a.lse[lidx] * kLog2e;
  }
}

// dQ^T += K^T dS^T from the stored dS: one workgroup per (64-query tile,
// batch, head), heaviest causal tile first.  The waves split the output dims
// (wave w: 16-dim blocks w + 4j) and each takes all 64 queries, so a K^T
// fragment feeds four MFMAs (16x16x32, all 32 keys of a tile) and each wave
// reads a quarter of K^T.  Per 32-key tile the K tile (row-major, the Row16
// swizzle) and the tile's four dS blocks (4 KiB, copied as they are) go
// HBM -> LDS through a 2-stage ring.
// dS blocks (ds, ds_nq32, ds_nk16): block (query block q/32, key block k/16)
// of a query head is 64 lanes x 16 bytes; lane 16*qd + c holds key c of the
// block and queries 4qd + [0,4) then 16 + 4qd + [0,4) (two 8-byte words).
// The dS^T operand of query block qb (16 queries) takes, in k-slot 8qd + j,
// key 16(j/4) + 4qd + j%4 (the order of Offs16::trans): two transposing reads
// (ds_read_b64_tr_b16) of the words of keys 4qd + s/4 (+16) and queries
// 4*(s%4) + [0,4) of the query block, addressed by lane s of each 16-lane
// group.  A query block at or past the valid queries was not stored and
// enters as zeros.
template <typename E, int D>
__global__ __launch_bounds__(kThreads, (D <= 256 ? 2 : 1)) void wide_bwd_dq_ds_kernel(WideBwdArgs ba) {
  const FlashArgs& a = ba.f;
  using OK = Offs16<E, D>;
  using RK = Row16<D>;
  constexpr int KT_B = RK::TILE_B, ST_B = 4096;
  constexpr int STAGE_B = KT_B + ST_B;
  constexpr int ND = D / 16, NJ = ND / 4;
  static_assert(ND % 4 == 0, "dims split evenly over the 4 waves");
  __shared__ __attribute__((aligned(1024))) unsigned char smem0[STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char smem1[STAGE_B];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, qd = lane >> 4;
  const int BH = a.B * a.Hq;
  const int n_qt = (a.Lq + kWQ - 1) / kWQ;
  const int bh = (int)blockIdx.x % BH;
  const int qt = n_qt - 1 - (int)blockIdx.x / BH;  // heaviest causal tile first
  const int b = bh / a.Hq, h = bh % a.Hq, hkv = h / (a.Hq / a.Hkv);
  const int q0 = qt * kWQ;
  const int q_hi = min(a.Lq, a.q_valid);
  int kv_end = min(a.Lk, a.kv_valid);
  if (a.kv_lengths) kv_end = min(kv_end, max(a.kv_lengths[b], 0));
  int kv_stop = kv_end;
  if (q0 >= q_hi) kv_stop = 0;
  else if (a.causal) kv_stop = min(kv_stop, min(q0 + kWQ, q_hi));
  const int n_tiles = (kv_stop + kWT - 1) / kWT;

  const uint32_t rowstride = (uint32_t)a.Hkv * 2 * D;
  const unsigned char* Kb = (const unsigned char*)a.k + ((size_t)b * a.Lk * a.Hkv + hkv) * (2 * D);
  // the dS blocks of query block 2qt + w/2, key block 2t + w%2: wave w's load
  const unsigned char* Sb = (const unsigned char*)(ba.ds + (((size_t)bh * ba.ds_nq32 + 2 * qt + (w >> 1)) *
                                                                ba.ds_nk16 + (w & 1)) * 512);
  OK ok;
  ok.init(lane, w, rowstride);
  // transposing K^T reads of this wave's dim blocks w + 4j (Offs16::trans)
  uint32_t offk[NJ];
  {
    const int rl = 4 * qd + (c >> 2), bsel = (c & 3) >> 1;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int i = w + 4 * j;
      offk[j] = 16 * RK::G * (i / OK::PT) + rl * RK::ROWB + 16 * ((2 * (i % OK::PT) + bsel) ^ RK::swz(rl)) + 8 * (c & 1);
    }
  }
  // dS^T reads: query block qb, keys 4qd + c/4 (lo: block 2(qb/2)), + 16 (hi:
  // the next key block); byte of the word: slot 16*(c%4) + 4qd + c/4, half qb%2
  uint32_t offs[4];
  {
    const int slot = 16 * (c & 3) + 4 * qd + (c >> 2);
#pragma unroll
    for (int qb = 0; qb < 4; ++qb) offs[qb] = KT_B + 1024 * (2 * (qb >> 1)) + 16 * slot + 8 * (qb & 1);
  }
  bool stored[4];
#pragma unroll
  for (int qb = 0; qb < 4; ++qb) stored[qb] = q0 + 32 * (qb >> 1) < q_hi;

  // acc[j][qb] = dQ^T[dims 16(w + 4j) + 4qd + r][query q0 + 16qb + c]
  f32x4 acc[NJ][4];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int qb = 0; qb < 4; ++qb) acc[j][qb] = f32x4{};

  auto issue = [&](int t, unsigned char* st) {
    const int k0 = t * kWT;
    ok.load(st, Kb + (size_t)k0 * rowstride, rowstride, min(kWT, kv_stop - k0), w);
    const rsrc_t rs = make_rsrc(Sb + (size_t)t * 2048, 1024);
    buffer_load_lds16_nt(rs, st + KT_B + 1024 * w, 16 * lane);  // dS is read once
  };

  auto compute = [&](const unsigned char* st) {
    typename E::v8 dsf[4];
#pragma unroll
    for (int qb = 0; qb < 4; ++qb) {
      const u32x2 lo = lds_read_tr16(st + offs[qb]);
      const u32x2 hi = lds_read_tr16(st + offs[qb] + 1024);
      dsf[qb] = stored[qb] ? E::as8(u32x4{lo[0], lo[1], hi[0], hi[1]}) : E::as8(u32x4{0u, 0u, 0u, 0u});
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const u32x2 lo = lds_read_tr16(st + offk[j]);
      const u32x2 hi = lds_read_tr16(st + offk[j] + 16 * RK::ROWB);
      const typename E::v8 kt = E::as8(u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
      for (int qb = 0; qb < 4; ++qb) acc[j][qb] = E::mma16(kt, dsf[qb], acc[j][qb]);
    }
  };

  if (n_tiles > 0) issue(0, smem0);
  for (int t = 0; t < n_tiles; t += 2) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t + 1 < n_tiles) issue(t + 1, smem1);
    compute(smem0);
    if (t + 1 >= n_tiles) break;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t + 2 < n_tiles) issue(t + 2, smem0);
    compute(smem1);
  }

#pragma unroll
  for (int qb = 0; qb < 4; ++qb) {
    const int qi = q0 + 16 * qb + c;
    if (qi >= a.Lq) continue;
    uint16_t* drow = (uint16_t*)ba.dq + ((size_t)(b * a.Lq + qi) * a.Hq + h) * D;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const u32x2 pk = {E::pack2(acc[j][qb][0], acc[j][qb][1]), E::pack2(acc[j][qb][2], acc[j][qb][3])};
      *(u32x2*)(drow + 16 * (w + 4 * j) + 4 * qd) = pk;
    }
  }
}

// Sums the head-group partials in split order and rounds to the 16-bit format:
// out[e] = sum_s part[s][e] for e < n (n a multiple of 4).
template <typename E>
__global__ __launch_bounds__(256) void wide_bwd_reduce_kernel(const float* part, int nsplit, size_t n,
                                                                uint16_t* out) {
  const size_t e = 4 * ((size_t)blockIdx.x * 256 + threadIdx.x);
  if (e >= n) return;
  f32x4 acc = *(const f32x4*)(part + e);
  for (int s = 1; s < nsplit; ++s) acc += *(const f32x4*)(part + (size_t)s * n + e);
  const u32x2 pk = {E::pack2(acc[0], acc[1]), E::pack2(acc[2], acc[3])};
  *(u32x2*)(out + e) = pk;
}

// ---------------------------------------------------------------------------
// Launch.
// ---------------------------------------------------------------------------
size_t wide_bwd_workspace(int64_t B, int64_t Hq, int64_t Lq, int64_t Lk, int64_t Hkv, int64_t D,
                          int64_t DV, int nsplit, bool shared) {
  size_t bytes = 8 * (size_t)B * Hq * Lq;
  bytes = (bytes + 255) & ~(size_t)255;
  if (nsplit > 1) bytes += (size_t)nsplit * B * Lk * Hkv * (D + (shared ? 0 : DV)) * 4;
  return bytes;
}

// Query-head groups per KV head for the dK/dV kernel: split the group (into
// a divisor of G) until the grid holds about 512 workgroups, two per CU of an
// MI355X.  A function of the shapes only, so that the workspace size is known
// without a device.
int wide_bwd_nsplit(int64_t B, int64_t Lk, int64_t Hq, int64_t Hkv) {
  const int64_t G = Hq / Hkv;
  const int64_t base = ((Lk + kWK - 1) / kWK) * B * Hkv;
  int ns = 1;
  while (base * ns < 512 && ns < G) {
    int next = ns + 1;
    while (next <= G && G % next) ++next;
    if (next > G) break;
    ns = next;
  }
  return ns;
}

template <typename E, int D, int DV, bool SHARED>
static int run_wide_bwd_t(WideBwdArgs& ba, hipStream_t s, const char* who, bool dq_only) {
  const FlashArgs& a = ba.f;
  const bool hb = a.bias != nullptr, db = ba.dbias != nullptr, ext = a.ext != 0;
  const long dq_blocks = (long)((a.Lq + kWQ - 1) / kWQ) * a.B * a.Hq;
  const long kv_blocks = (long)((a.Lk + kWK - 1) / kWK) * a.B * a.Hkv * ba.nsplit;
  if (dq_blocks > 0x7fffffffL || kv_blocks > 0x7fffffffL) return fail(PJX_ERR_INVALID, "wide backward: grid too large");
  const dim3 blk(kThreads);
  // the dS route: head dim 256 only (at the latent widths the key-side kernel
  // with the store ran at half its speed, more than the dQ kernel saves)
  if constexpr (!SHARED) {
   if (ba.ds && !hb && !db && !ext && !dq_only) {
    // the dS route: delta, dK/dV (dC) storing dS, the partial sum, dQ from dS
    const long rows = (long)a.B * a.Lq * a.Hq;
    launch_kernel<wide_bwd_delta_kernel<E, DV>>(dim3((unsigned)((rows + kThreads / 4 - 1) / (kThreads / 4))), blk, 0, s,
                                                ba);
    int rc = check_launch(who);
    if (rc != PJX_OK) return rc;
    if (kv_blocks > 0) {
      launch_kernel<wide_bwd_dc_ds_kernel<E, D, DV, SHARED>>(dim3((unsigned)kv_blocks), blk, 0, s, ba);
      rc = check_launch(who);
      if (rc != PJX_OK) return rc;
    }
    if (ba.nsplit > 1) {
      const size_t nk = (size_t)a.B * a.Lk * a.Hkv * D;
      launch_kernel<wide_bwd_reduce_kernel<E>>(dim3((unsigned)((nk / 4 + 255) / 256)), dim3(256), 0, s,
                         (const float*)ba.part, ba.nsplit, nk, (uint16_t*)ba.dk);
      if constexpr (!SHARED) {
        const size_t nv = (size_t)a.B * a.Lk * a.Hkv * DV;
        launch_kernel<wide_bwd_reduce_kernel<E>>(dim3((unsigned)((nv / 4 + 255) / 256)), dim3(256), 0, s,
                           (const float*)(ba.part + (size_t)ba.nsplit * nk), ba.nsplit, nv, (uint16_t*)ba.dv);
      }
      rc = check_launch(who);
      if (rc != PJX_OK) return rc;
    }
    launch_kernel<wide_bwd_dq_ds_kernel<E, D>>(dim3((unsigned)dq_blocks), blk, 0, s, ba);
    return check_launch(who);
   }
  }
#define PJX_DQ(BI, EX) launch_kernel<wide_bwd_dq_kernel<E, D, DV, SHARED, BI, EX>>(dim3((unsigned)dq_blocks), blk, 0, s, ba)
  if (ext) {
    if (db) PJX_DQ(2, 2); else if (hb) PJX_DQ(1, 2); else PJX_DQ(0, 2);
  } else {
    if (db) PJX_DQ(2, 0); else if (hb) PJX_DQ(1, 0); else PJX_DQ(0, 0);
  }
#undef PJX_DQ
  int rc = check_launch(who);
  if (rc != PJX_OK || dq_only) return rc;
  if (kv_blocks > 0) {
#define PJX_KV(BI, EX) launch_kernel<wide_bwd_dkdv_kernel<E, D, DV, SHARED, BI, EX>>(dim3((unsigned)kv_blocks), blk, 0, s, ba)
    if (ext) {
      if (hb) PJX_KV(true, 2); else PJX_KV(false, 2);
    } else if (hb) {
      PJX_KV(true, 0);
    } else {
      launch_kernel<wide_bwd_dc_kernel<E, D, DV, SHARED>>(dim3((unsigned)kv_blocks), blk, 0, s, ba);
    }
#undef PJX_KV
    rc = check_launch(who);
    if (rc != PJX_OK) return rc;
  }
  if (ba.nsplit > 1) {
    const size_t nk = (size_t)a.B * a.Lk * a.Hkv * D;
    launch_kernel<wide_bwd_reduce_kernel<E>>(dim3((unsigned)((nk / 4 + 255) / 256)), dim3(256), 0, s,
                       (const float*)ba.part, ba.nsplit, nk, (uint16_t*)ba.dk);
    if constexpr (!SHARED) {
      const size_t nv = (size_t)a.B * a.Lk * a.Hkv * DV;
      launch_kernel<wide_bwd_reduce_kernel<E>>(dim3((unsigned)((nv / 4 + 255) / 256)), dim3(256), 0, s,
                         (const float*)(ba.part + (size_t)ba.nsplit * nk), ba.nsplit, nv, (uint16_t*)ba.dv);
    }
    rc = check_launch(who);
  }
  return rc;
}

template <typename E>
static int run_wide_bwd_fmt(WideBwdArgs& ba, int D, int DV, bool shared, hipStream_t s, const char* who,
                            bool dq_only) {
  if (!shared && D == 256 && DV == 256) return run_wide_bwd_t<E, 256, 256, false>(ba, s, who, dq_only);
  if (shared && D == 576 && DV == 512) return run_wide_bwd_t<E, 576, 512, true>(ba, s, who, dq_only);
  if (shared && D == 576 && DV == 576) return run_wide_bwd_t<E, 576, 576, true>(ba, s, who, dq_only);
  if (shared && D == 512 && DV == 512) return run_wide_bwd_t<E, 512, 512, true>(ba, s, who, dq_only);
  return fail(PJX_ERR_INVALID, "wide backward: unsupported head widths");
}

int run_wide_bwd(WideBwdArgs& ba, int D, int DV, bool shared, hipStream_t s, const char* who, bool dq_only) {
  return ba.f.f16 ? run_wide_bwd_fmt<F16Fmt>(ba, D, DV, shared, s, who, dq_only)
                  : run_wide_bwd_fmt<Bf16Fmt>(ba, D, DV, shared, s, who, dq_only);
}

}  // namespace pjx

using namespace pjx;

extern "C" size_t pjx_mla_bwd_workspace_size(int64_t batch, int64_t heads, int64_t q_len,
                                             int64_t kv_len, int64_t rank) {
  if (batch <= 0 || heads <= 0 || q_len < 0 || kv_len < 0 || rank <= 0) return 0;
  return wide_bwd_workspace(batch, heads, q_len, kv_len, 1, rank, 0,
                            wide_bwd_nsplit(batch, kv_len, heads, 1), true);
}

namespace pjx {
static_assert(kWQ == 64 && kWK == 64, "the dS block counts of flash_common.h follow these tiles");
size_t wide_bwd_ds_bytes(int64_t B, int64_t Hq, int64_t Lq, int64_t Lk) {
  const int64_t nq32 = wide_bwd_ds_nq32(Lq), nk16 = wide_bwd_ds_nk16(Lk);
  return (size_t)B * Hq * nq32 * nk16 * 1024;
}
}  // namespace pjx

extern "C" int pjx_mla_bwd(int dtype, const void* q, const void* cache, const void* o,
                           const void* dout, const float* lse, void* dq, void* dcache,
                           void* workspace, size_t workspace_bytes, const int32_t* kv_lengths,
                           const float* bias, int64_t bias_batch, int64_t bias_heads, int64_t batch,
                           int64_t q_len, int64_t kv_len, int64_t heads, int64_t rank,
                           int64_t v_dim, int64_t q_valid, int64_t kv_valid, int causal,
                           float sm_scale, const pjx_score_mods* mods, void* stream) {
  clear_error();
  const char* who = "pjx_mla_bwd";
  if (dtype != PJX_DTYPE_BF16 && dtype != PJX_DTYPE_F16)
    return fail(PJX_ERR_INVALID, "pjx_mla_bwd: dtype must be PJX_DTYPE_BF16 or PJX_DTYPE_F16");
  if (!((rank == 576 && (v_dim == 512 || v_dim == 576)) || (rank == 512 && v_dim == 512)))
    return fail(PJX_ERR_INVALID, "pjx_mla_bwd: (rank, v_dim) must be (576, 512), (576, 576) or (512, 512)");
  // zero-element tensors may come as null pointers
  const bool q_none = batch == 0 || q_len == 0, k_none = batch == 0 || kv_len == 0;
  if ((!q_none && (!q || !o || !dout || !lse || !dq)) || (!k_none && (!cache || !dcache)))
    return fail(PJX_ERR_INVALID, "pjx_mla_bwd: q, cache, o, dout, lse, dq, dcache must be non-null");
  if (batch < 0 || q_len < 0 || kv_len < 0 || heads <= 0)
    return fail(PJX_ERR_INVALID, "pjx_mla_bwd: negative or zero size");
  if (!(sm_scale > 0.f)) return fail(PJX_ERR_INVALID, "pjx_mla_bwd: sm_scale must be > 0");
  if (bias && !((bias_batch == 1 || bias_batch == batch) && (bias_heads == 1 || bias_heads == heads)))
    return fail(PJX_ERR_INVALID, "pjx_mla_bwd: bias must be [1|B, 1|H, Lq, S]");
  if (batch * q_len * heads * rank > ((int64_t)1 << 40) || q_len > (1 << 30) || kv_len > (1 << 30) ||
      batch * kv_len * rank * 4 * heads > ((int64_t)1 << 46))
    return fail(PJX_ERR_INVALID, "pjx_mla_bwd: sizes out of range");
  if (batch == 0 || (q_len == 0 && kv_len == 0)) return PJX_OK;
  if (kv_len == 0) return zero_u16(dq, (size_t)(batch * q_len * heads * rank), (hipStream_t)stream, who);
  if (q_len == 0) return zero_u16(dcache, (size_t)(batch * kv_len * rank), (hipStream_t)stream, who);
  const int nsplit = wide_bwd_nsplit(batch, kv_len, heads, 1);
  const size_t need = wide_bwd_workspace(batch, heads, q_len, kv_len, 1, rank, 0, nsplit, true);
  if (!workspace || workspace_bytes < need)
    return fail(PJX_ERR_WORKSPACE, "pjx_mla_bwd: workspace missing or smaller than pjx_mla_bwd_workspace_size()");
  WideBwdArgs ba;
  FlashArgs& a = ba.f;
  a.q = q; a.k = cache; a.v = cache; a.o = const_cast<void*>(o); a.lse = const_cast<float*>(lse);
  a.kv_lengths = kv_lengths;
  a.bias = bias;
  a.bias_hstride = (bias && bias_heads != 1) ? q_len * kv_len : 0;
  a.bias_bstride = (bias && bias_batch != 1) ? bias_heads * q_len * kv_len : 0;
  a.B = (int)batch; a.Lq = (int)q_len; a.Lk = (int)kv_len;
  a.Hq = (int)heads; a.Hkv = 1;
  a.q_valid = (int)std::min<int64_t>(std::max<int64_t>(q_valid, 0), q_len);
  a.kv_valid = (int)std::min<int64_t>(std::max<int64_t>(kv_valid, 0), kv_len);
  a.causal = causal ? 1 : 0;
  a.f16 = dtype == PJX_DTYPE_F16;
  a.scale = sm_scale;
  a.n_qtiles = (int)((q_len + kBQ - 1) / kBQ);
  a.dv = (int)v_dim;
  const int mrc = lower_score_mods(mods, a, who);
  if (mrc != PJX_OK) return mrc;
  ba.dout = dout;
  ba.delta = (float*)workspace;
  ba.lse2 = ba.delta + batch * heads * q_len;
  ba.part = (float*)((unsigned char*)workspace + ((8 * (size_t)batch * heads * q_len + 255) & ~(size_t)255));
  ba.nsplit = nsplit;
  ba.dq = dq;
  ba.dk = dcache;
  ba.dv = nullptr;
  ba.dbias = nullptr;
  ba.ds = nullptr;  // the latent keeps the two-kernel route
  ba.ds_nq32 = ba.ds_nk16 = 0;
  return run_wide_bwd(ba, (int)rank, (int)v_dim, true, (hipStream_t)stream, who);
}
