// Flash-attention forward for gfx950, bf16 / fp16 with a dense fp32 bias: the LDS
// ring kernel (semantics as flash_fwd.hip's kernels: scores sm_scale * q.k in
// fp32, then the bias, then the mask; probjax's XLA attention reference,
// probjax/nn/pallas_kernels/kernels/attention_xla.py:339-429, with DenseBias
// from attention_mask_bias.py:1807-1922).
//
// Built with -mllvm -amdgpu-mfma-vgpr-form=1 (probjax_amd/build.py), which
// keeps the MFMA accumulators in VGPRs, where the softmax reads them
// directly; in AGPRs every score is copied out first (measured on the
// one-wave-per-SIMD form of this kernel: C4 48.5 -> 44.1 us on MI355X).
#include "flash_common.h"

namespace pjx {

// ---------------------------------------------------------------------------
// bf16 path with a dense fp32 bias, streamed through LDS.  The bias is the
// bulk of the bytes (4 B per score against 4*D bytes of K/V per key shared by
// 128 queries), and per score the kernel adds it and runs the softmax: at
// D = 64 the VALU work per score outweighs the MFMA work.  So G groups of 4
// waves share the 128 queries of a workgroup: waves w, w+4 (and w+8) share a
// SIMD, group j takes the 32-key tiles t with t % G == j, each wave with its
// own online softmax for its 32 rows, and the waves of a SIMD interleave
// their MFMAs, exponentials and LDS reads (with 4 waves, one per SIMD at one
// workgroup per CU, nothing overlaps them).  G = 2, or 3 at D = 64 for key
// lengths up to 2048, where the third wave per SIMD hides more latency than
// the shallower ring costs.
//
// Ring: a set of G tiles (one per group) is one step.  NP set slots of G
// stages each (K | V | bias block [128 queries][32 keys] per stage), all
// copied by buffer->LDS loads, NP-1 sets in flight while one is computed;
// each group loads its own tile of a set, a quarter per wave.  Bias rows
// (128 B) keep their 16-byte chunks XOR-swizzled by bias_swz(row), the D = 64
// K rows' swizzle, for the same read pattern (lane l reads a chunk of row
// l%32).  Every path
// issues the same loads in the same order (tiles past the last one read
// nothing) and the loop has no early exit, so waits are partial vmcnt counts
// the compiler can see through; one barrier per set (after the wait for the
// next set, before its slot is reloaded), built from s_barrier and wavefront
// fences so it does not wait for the sets in flight.  At the end groups
// 1 .. G-1 hand (max, sum, O) to group 0 through LDS; group 0 merges them and
// writes the rows.  The products and the softmax are those of flash_fwd_bf16_kernel.
// Requires Lk % 4 == 0 (16-byte bias chunks) and Lq*Lk*4 < 2^31 (32-bit
// buffer offsets within one (batch, head) bias slice).
// ---------------------------------------------------------------------------
// Chunk swizzle of the 128-byte bias rows in LDS (8 chunks of 4 keys).
__device__ __forceinline__ int bias_swz(int r) { return (r & 6) | ((r >> 3) & 1); }

template <int D, int G_>
struct BiasRing {
  using T = Bf16Tile<D, 32>;
  static constexpr int G = G_;                            // groups of 4 waves
  static constexpr int BIAS_ROWB = 32 * 4;                // 32 keys of fp32
  static constexpr int BIAS_B = kBQ * BIAS_ROWB;          // 16 KiB
  static constexpr int STAGE_B = 2 * T::TILE_B + BIAS_B;  // K | V | bias
  static constexpr int SET_B = G * STAGE_B;  // one set: a stage per group
  static constexpr int NP = (3 * SET_B <= 150 * 1024) ? 3 : 2;
  static constexpr int NLB = BIAS_B / (4 * 1024);         // bias loads per wave per tile
  static constexpr int NL = 2 * T::NLD + NLB;             // loads per wave per set
  static_assert(NL * (NP - 1) < 64, "vmcnt range");
  static_assert(NP >= 2, "ring depth");
  static_assert(NP * SET_B <= 150 * 1024, "LDS");
};

template <typename E, int D, int G_>
__global__ __launch_bounds__(G_ * kThreads, 1) void flash_fwd_bf16_bias_ring_kernel(FlashArgs a) {
  using T = Bf16Tile<D, 32>;
  using R = BiasRing<D, G_>;
  constexpr int BK = 32, ROWB = T::ROWB, TILE_B = T::TILE_B, NP = R::NP, NL = R::NL, G = R::G;
  constexpr int BROWB = R::BIAS_ROWB, STAGE_B = R::STAGE_B;
  static_assert(T::BK == BK, "32-key tiles");
  __shared__ __attribute__((aligned(1024))) unsigned char ps0[R::SET_B];
  __shared__ __attribute__((aligned(1024))) unsigned char ps1[R::SET_B];
  __shared__ __attribute__((aligned(1024))) unsigned char ps2[NP > 2 ? R::SET_B : 1024];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w8 = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = w8 >> 2, w = w8 & 3;  // tile group (tiles t with t % G == grp), wave within it
  BlockGeom g = block_geom(a);
  g.qw = __builtin_amdgcn_readfirstlane(g.q0 + 32 * w);
  g.qi = g.qw + (tid & 31);
  const int col = lane & 31, half = lane >> 5;
  const uint32_t rowstride = (uint32_t)a.Hkv * D * 2;
  const unsigned char* Kb = (const unsigned char*)a.k + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * ROWB;
  const unsigned char* Vb = (const unsigned char*)a.v + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * ROWB;
  const float* bslice = a.bias + (size_t)g.b * a.bias_bstride + (size_t)g.h * a.bias_hstride;
  const uint32_t slice_bytes = (uint32_t)a.Lq * (uint32_t)a.Lk * 4u;
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

  // K/V rows 8w + .. of the group's tile; bias rows 32w + 8j + lane/8, LDS
  // chunk lane%8 from global chunk (lane%8) ^ bias_swz(row).
  uint32_t voffK[T::NLD], voffV[T::NLD];
#pragma unroll
  for (int j = 0; j < T::NLD; ++j) {
    const int r = 8 * w + T::RPI * j + lane / T::NC, slot = lane % T::NC;
    voffK[j] = r * rowstride + 16 * (slot ^ T::swz_k(r));
    voffV[j] = r * rowstride + 16 * (slot ^ T::swz_v(r));
  }
  uint32_t voffB[R::NLB];
#pragma unroll
  for (int j = 0; j < R::NLB; ++j) {
    const int r = 32 * w + 8 * j + lane / 8, slot = lane % 8;
    voffB[j] = (uint32_t)(g.q0 + r) * (uint32_t)a.Lk * 4u + 16u * (uint32_t)(slot ^ bias_swz(r));
  }
  uint32_t offK[D / 16];
#pragma unroll
  for (int st = 0; st < D / 16; ++st) offK[st] = col * ROWB + 16 * ((2 * st + half) ^ T::swz_k(col));
  uint32_t offV[D / 32];
  {
    const int s16 = lane & 15, gq4 = lane >> 4;
    const int r = 4 * half + s16 / 4;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int chunk = 4 * db + 2 * (gq4 & 1) + ((s16 & 3) >> 1);
      offV[db] = r * ROWB + 16 * (chunk ^ T::swz_v(r)) + 8 * (s16 & 1);
    }
  }
  const int brow_l = 32 * w + col;
  const uint32_t offB = brow_l * BROWB;

  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16{};
  float m_run = kMaxInit, l_run = 0.f;

  const int n_tiles = (g.kv_stop + BK - 1) / BK;
  const int n_sets = (n_tiles + G - 1) / G;
  const int q_last_w = g.qw + 31;
  const float cx = kLog2e;

  // This group's tile of set p into its stage of the set's slot.
  auto issue = [&](int p, unsigned char* slot) {
    const int k0 = (G * p + grp) * BK;
    unsigned char* ks = slot + grp * STAGE_B;
    const int nvalid = max(0, min(BK, g.kv_stop - k0));
    const uint32_t kvbytes =
        __builtin_amdgcn_readfirstlane(nvalid > 0 ? (uint32_t)(nvalid - 1) * rowstride + ROWB : 0u);
    const rsrc_t rk = make_rsrc(Kb + (size_t)max(k0, 0) * rowstride, kvbytes);
    const rsrc_t rv = make_rsrc(Vb + (size_t)max(k0, 0) * rowstride, kvbytes);
#pragma unroll
    for (int j = 0; j < T::NLD; ++j) {
      const int r0 = 8 * w + T::RPI * j;
      buffer_load_lds16(rk, ks + r0 * ROWB, voffK[j]);
      buffer_load_lds16(rv, ks + TILE_B + r0 * ROWB, voffV[j]);
    }
    const uint32_t bbytes = __builtin_amdgcn_readfirstlane(nvalid > 0 ? slice_bytes : 0u);
    const rsrc_t rb = make_rsrc(bslice, bbytes);
#pragma unroll
    for (int j = 0; j < R::NLB; ++j)
      buffer_load_lds16(rb, ks + 2 * TILE_B + (32 * w + 8 * j) * BROWB, voffB[j] + (uint32_t)k0 * 4u);
  };

  auto compute = [&](int p, const unsigned char* slot) {
    const int k0 = (G * p + grp) * BK;
    if (k0 >= g.kv_stop) return;            // past the last tile
    if (a.causal && k0 > q_last_w) return;  // tile above this wave's diagonal
    const unsigned char* ks = slot + grp * STAGE_B;
    const unsigned char* vs = ks + TILE_B;
    const unsigned char* bs = ks + 2 * TILE_B;

    f32x16 s = f32x16{};
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
      const typename E::v8 kf = E::as8(*(const u32x4*)(ks + offK[st]));
      s = E::mma32(kf, qf[st], s);
    }
    // Register r holds key k0 + 8*(r/4) + 4*half + r%4: bias chunk
    // 2*(r/4) + half of this lane's row.
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const f32x4 bv = *(const f32x4*)(bs + offB + 16 * ((2 * gq + half) ^ bias_swz(brow_l)));
#pragma unroll
      for (int j = 0; j < 4; ++j) s[4 * gq + j] = fmaf(s[4 * gq + j], a.scale, bv[j]);
    }
    const bool need_mask = (k0 + BK > g.kv_end) || (a.causal && k0 + BK - 1 > g.qw) ||
                           (g.qw + 31 >= g.q_hi);
    if (need_mask) {
      const int base = k0 + 4 * half;
      int lim = g.kv_end - 1 - base;
      if (a.causal) lim = min(lim, g.qi - base);
      if (!row_ok) lim = -1;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + (r & 3) > lim) s[r] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; r += 2) mx = fmaxf(mx, fmaxf(s[r], s[r + 1]));
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
    for (int r = 0; r < 16; ++r) {
      const float pv = fast_exp2(fmaf(s[r], cx, -m_run));
      rs += pv;
      s[r] = pv;
    }
    l_run += rs;
    typename E::v8 pf[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      u32x4 pk;
#pragma unroll
      for (int j = 0; j < 4; ++j) pk[j] = E::pack2(s[8 * c + 2 * j], s[8 * c + 2 * j + 1]);
      pf[c] = E::as8(pk);
    }
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const u32x2 lo = lds_read_tr16(vs + 16 * c * ROWB + offV[db]);
        const u32x2 hi = lds_read_tr16(vs + (16 * c + 8) * ROWB + offV[db]);
        const u32x4 av = {lo[0], lo[1], hi[0], hi[1]};
        acc[db] = E::mma32(E::as8(av), pf[c], acc[db]);
      }
    }
  };

  // Set p lives in slot p % NP.  Before computing set p its loads have
  // landed for every wave; after, wait for set p+1, one barrier, then set
  // p+NP is loaded into slot p % NP.
  issue(0, ps0);
  wait_vmcnt<NL>();  // q's loads (issued before set 0's) have landed
  issue(1, ps1);
  if constexpr (NP > 2) issue(2, ps2);
  wait_vmcnt<(NP - 1) * NL>();
  stage_barrier();
  for (int p = 0; p < n_sets; p += NP) {
    compute(p, ps0);
    wait_vmcnt<(NP - 2) * NL>();
    stage_barrier();
    issue(p + NP, ps0);
    compute(p + 1, ps1);
    wait_vmcnt<(NP - 2) * NL>();
    stage_barrier();
    issue(p + NP + 1, ps1);
    if constexpr (NP > 2) {
      compute(p + 2, ps2);
      wait_vmcnt<(NP - 2) * NL>();
      stage_barrier();
      issue(p + NP + 2, ps2);
    }
  }
  wait_vmcnt<0>();
  stage_barrier();  // every wave is done with the ring

  // Groups 1 .. G-1 hand their (max, sum, O) to group 0 through LDS, lane by
  // lane in the same register layout: O as 16-byte quads [group-1][D/32 * 4]
  // [4 waves][64 lanes] in set slot 0 (consecutive lanes, consecutive banks),
  // (max, sum) in slot 1.
  constexpr int QUADS = (D / 32) * 4;
  static_assert((G - 1) * QUADS * 256 * 16 <= R::SET_B && (G - 1) * 256 * 8 <= R::SET_B, "hand-off fits");
  if (grp > 0) {
    f32x4* xo = (f32x4*)ps0 + ((grp - 1) * QUADS) * 256 + w * 64 + lane;
    float* xml = (float*)ps1 + 2 * ((grp - 1) * 256 + w * 64 + lane);
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
      for (int r = 0; r < 16; r += 4)
        xo[(4 * i + r / 4) * 256] = f32x4{acc[i][r], acc[i][r + 1], acc[i][r + 2], acc[i][r + 3]};
    xml[0] = m_run;
    xml[1] = l_run;
  }
  stage_barrier();
  if (grp > 0) return;
  float mg[G], lg[G], fg[G];
  mg[0] = m_run;
  lg[0] = l_run;
  float M = m_run;
#pragma unroll
  for (int gi = 1; gi < G; ++gi) {
    const float* xml = (const float*)ps1 + 2 * ((gi - 1) * 256 + w * 64 + lane);
    mg[gi] = xml[0];
    lg[gi] = xml[1];
    M = fmaxf(M, mg[gi]);
  }
  float lsum = 0.f;
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    fg[gi] = fast_exp2(mg[gi] - M);
    lsum = fmaf(lg[gi], fg[gi], lsum);
  }
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int r = 0; r < 16; r += 4) {
      f32x4 o = {acc[i][r] * fg[0], acc[i][r + 1] * fg[0], acc[i][r + 2] * fg[0], acc[i][r + 3] * fg[0]};
#pragma unroll
      for (int gi = 1; gi < G; ++gi) {
        const f32x4 o1 = ((const f32x4*)ps0)[((gi - 1) * QUADS + 4 * i + r / 4) * 256 + w * 64 + lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = fmaf(o1[j], fg[gi], o[j]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][r + j] = o[j];
    }
  const float l_tot = xor32_sum(lsum);
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
      a.lse[((size_t)g.b * a.Hq + g.h) * a.Lq + g.qi] = l_tot > 0.f ? (M + __log2f(l_tot)) * kLn2 : INFINITY;
  }
}

constexpr int kBiasRing3MaxKeys = 2048;

template <typename E>
static void launch_ring(int head_dim, const FlashArgs& a, hipStream_t stream) {
  const long blocks = (long)a.n_qtiles * a.B * a.Hq;
  if (head_dim == 128)
    launch_kernel<flash_fwd_bf16_bias_ring_kernel<E, 128, 2>>(dim3((unsigned)blocks), dim3(2 * kThreads), 0,
                       stream, a);
  else if (a.Lk <= kBiasRing3MaxKeys)
    launch_kernel<flash_fwd_bf16_bias_ring_kernel<E, 64, 3>>(dim3((unsigned)blocks), dim3(3 * kThreads), 0,
                       stream, a);
  else
    launch_kernel<flash_fwd_bf16_bias_ring_kernel<E, 64, 2>>(dim3((unsigned)blocks), dim3(2 * kThreads), 0,
                       stream, a);
}

int launch_flash_bias_ring(int head_dim, const FlashArgs& a, hipStream_t stream) {
  if (a.f16)
    launch_ring<F16Fmt>(head_dim, a, stream);
  else
    launch_ring<Bf16Fmt>(head_dim, a, stream);
  return check_launch("pjx_flash_fwd");
}

}  // namespace pjx
