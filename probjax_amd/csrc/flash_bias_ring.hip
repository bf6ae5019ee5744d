// Flash-attention forward for gfx950, bf16 with a dense fp32 bias: the LDS
// ring kernel (semantics as flash_fwd.hip's kernels: scores sm_scale * q.k in
// fp32, then the bias, then the mask; probjax's XLA attention reference,
// probjax/nn/pallas_kernels/kernels/attention_xla.py:339-429, with DenseBias
// from attention_mask_bias.py:1807-1922).
//
// Built with -mllvm -amdgpu-mfma-vgpr-form=1 (probjax_amd/build.py): the
// kernel's LDS ring allows one wave per SIMD, and at that occupancy the
// compiler otherwise puts the MFMA accumulators in AGPRs and copies every
// score out of them for the softmax; in VGPRs the softmax reads them directly
// (C4: 48.5 -> 44.1 us on MI355X).
#include "flash_common.h"

namespace pjx {

// ---------------------------------------------------------------------------
// bf16 path with a dense fp32 bias, streamed through LDS.  The bias is the
// bulk of the bytes (4 B per score against 4*D bytes of K/V per key shared by
// 128 queries), so the kernel is a streaming kernel: each stage of an NS-deep
// LDS ring holds one tile's K, V and bias block [128 queries][64 keys], all
// copied by buffer->LDS loads, and NS-1 tiles are in flight while one is
// computed (one workgroup per CU).  Bias rows (256 B) keep their 16-byte
// chunks XOR-swizzled by (row & 15), so the 16 lanes reading one chunk of 16
// rows hit distinct banks.  The products and the softmax are those of
// flash_fwd_bf16_kernel.
//
// Ring protocol: every path issues the same loads in the same order (tiles
// past the last one read nothing) and the loop has no early exit, so waits
// are partial vmcnt counts the compiler can see through; one barrier per tile
// (after the wait for the next tile, before its stage is reloaded), built from
// s_barrier and wavefront fences so it does not wait for the tiles in flight.
// Requires Lk % 4 == 0 (16-byte bias chunks) and Lq*Lk*4 < 2^31 (32-bit buffer
// offsets within one (batch, head) bias slice).
// ---------------------------------------------------------------------------
template <int D>
struct BiasRing {
  using T = Bf16Tile<D>;
  static constexpr int BIAS_ROWB = T::BK * 4;            // 64 keys of fp32
  static constexpr int BIAS_B = kBQ * BIAS_ROWB;          // 32 KiB
  static constexpr int STAGE_B = 2 * T::TILE_B + BIAS_B;  // K | V | bias
  static constexpr int NS = (3 * STAGE_B <= 150 * 1024) ? 3 : 2;
  static constexpr int NLB = BIAS_B / (4 * 1024);         // bias loads per wave per tile
  static constexpr int NL = 2 * T::NLD + NLB;             // all loads per wave per tile
  static_assert(NL * (NS - 1) < 64, "vmcnt range");
};

template <int D>
__global__ __launch_bounds__(kThreads, 1) void flash_fwd_bf16_bias_ring_kernel(FlashArgs a) {
  using T = Bf16Tile<D>;
  using R = BiasRing<D>;
  constexpr int BK = T::BK, ROWB = T::ROWB, TILE_B = T::TILE_B, NS = R::NS, NL = R::NL;
  constexpr int BROWB = R::BIAS_ROWB;
  __shared__ __attribute__((aligned(1024))) unsigned char st0[R::STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char st1[R::STAGE_B];
  __shared__ __attribute__((aligned(1024))) unsigned char st2[NS > 2 ? R::STAGE_B : 1024];

  BlockGeom g = block_geom(a);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  g.qw = __builtin_amdgcn_readfirstlane(g.qw);
  const int col = lane & 31, half = lane >> 5;
  const uint32_t rowstride = (uint32_t)a.Hkv * D * 2;
  const unsigned char* Kb = (const unsigned char*)a.k + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * ROWB;
  const unsigned char* Vb = (const unsigned char*)a.v + ((size_t)g.b * a.Lk * a.Hkv + g.hkv) * ROWB;
  const float* bslice = a.bias + (size_t)g.b * a.bias_bstride + (size_t)g.h * a.bias_hstride;
  const uint32_t slice_bytes = (uint32_t)a.Lq * (uint32_t)a.Lk * 4u;
  const bool row_in = g.qi < a.Lq;
  const bool row_ok = g.qi < g.q_hi;

  // Q^T as the B operand: lane holds query `col`, dims 16*s + 8*half + [0,8).
  bf16x8 qf[D / 16];
  {
    const uint16_t* qrow =
        (const uint16_t*)a.q + ((size_t)(g.b * a.Lq + (row_in ? g.qi : 0)) * a.Hq + g.h) * D;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row_in) raw = *(const u32x4*)(qrow + 16 * s + 8 * half);
      qf[s] = as_bf16x8(raw);
    }
  }

  // Per-lane offsets, fixed for the whole key loop.
  uint32_t voffK[T::NLD], voffV[T::NLD];
#pragma unroll
  for (int j = 0; j < T::NLD; ++j) {
    const int r = 16 * w + T::RPI * j + lane / T::NC, slot = lane % T::NC;
    voffK[j] = r * rowstride + 16 * (slot ^ T::swz_k(r));
    voffV[j] = r * rowstride + 16 * (slot ^ T::swz_v(r));
  }
  // Bias load j of wave w fills rows 32w + 4j + lane/16 of the block, LDS
  // chunk lane%16, from global chunk (lane%16) ^ (row & 15) of that row (the
  // tile's first key is added per tile).
  uint32_t voffB[R::NLB];
#pragma unroll
  for (int j = 0; j < R::NLB; ++j) {
    const int r = 32 * w + 4 * j + lane / 16, slot = lane % 16;
    voffB[j] = (uint32_t)(g.q0 + r) * (uint32_t)a.Lk * 4u + 16u * (uint32_t)(slot ^ (r & 15));
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
  const int brow_l = 32 * w + col;  // this lane's row of the bias block
  const uint32_t offB = brow_l * BROWB;

  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16{};
  float m_run = kMaxInit, l_run = 0.f;

  const int n_tiles = (g.kv_stop + BK - 1) / BK;
  const int q_last_w = g.qw + 31;
  const float cx = kLog2e;

  auto issue = [&](int t, unsigned char* ks) {
    const int k0 = t * BK;
    const int nvalid = max(0, min(BK, g.kv_stop - k0));
    // Scalar operands only (readfirstlane): a buffer descriptor built from a
    // vector-unit select would need a waterfall loop.
    const uint32_t kvbytes =
        __builtin_amdgcn_readfirstlane(nvalid > 0 ? (uint32_t)(nvalid - 1) * rowstride + ROWB : 0u);
    const rsrc_t rk = make_rsrc(Kb + (size_t)k0 * rowstride, kvbytes);
    const rsrc_t rv = make_rsrc(Vb + (size_t)k0 * rowstride, kvbytes);
#pragma unroll
    for (int j = 0; j < T::NLD; ++j) {
      const int r0 = 16 * w + T::RPI * j;
      buffer_load_lds16(rk, ks + r0 * ROWB, voffK[j]);
      buffer_load_lds16(rv, ks + TILE_B + r0 * ROWB, voffV[j]);
    }
    // The bias resource spans the (batch, head) slice; the tile's first key
    // is part of the per-lane offset, so the range check covers it: keys past
    // Lk read the next row's values (masked keys) or, past the slice, zeros.
    // Past the last tile the resource is empty and the loads read nothing.
    const uint32_t bbytes = __builtin_amdgcn_readfirstlane(nvalid > 0 ? slice_bytes : 0u);
    const rsrc_t rb = make_rsrc(bslice, bbytes);
#pragma unroll
    for (int j = 0; j < R::NLB; ++j)
      buffer_load_lds16(rb, ks + 2 * TILE_B + (32 * w + 4 * j) * BROWB, voffB[j] + (uint32_t)k0 * 4u);
  };

  auto compute = [&](int t, const unsigned char* ks) {
    const int k0 = t * BK;
    if (k0 >= g.kv_stop) return;            // past the last tile
    if (a.causal && k0 > q_last_w) return;  // tile above this wave's diagonal
    const unsigned char* vs = ks + TILE_B;
    const unsigned char* bs = ks + 2 * TILE_B;

    f32x16 s[BK / 32];
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb) {
      s[kb] = f32x16{};
#pragma unroll
      for (int st = 0; st < D / 16; ++st) {
        const bf16x8 kf = as_bf16x8(*(const u32x4*)(ks + kb * 32 * ROWB + offK[st]));
        s[kb] = mfma32x32x16(kf, qf[st], s[kb]);
      }
    }
    // Register r of block kb holds key k0 + kb*32 + 8*(r/4) + 4*half + r%4:
    // bias chunk 8*kb + 2*(r/4) + half of this lane's row.
#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const f32x4 bv = *(const f32x4*)(bs + offB + 16 * ((8 * kb + 2 * gq + half) ^ (brow_l & 15)));
#pragma unroll
        for (int j = 0; j < 4; ++j) s[kb][4 * gq + j] = fmaf(s[kb][4 * gq + j], a.scale, bv[j]);
      }
    const bool need_mask = (k0 + BK > g.kv_end) || (a.causal && k0 + BK - 1 > g.qw) ||
                           (g.qw + 31 >= g.q_hi);
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

    bf16x8 pf[BK / 16];
#pragma unroll
    for (int c = 0; c < BK / 16; ++c) {
      u32x4 pk;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        pk[j] = pack_bf16x2(s[c >> 1][8 * (c & 1) + 2 * j], s[c >> 1][8 * (c & 1) + 2 * j + 1]);
      pf[c] = as_bf16x8(pk);
    }
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
#pragma unroll
      for (int c = 0; c < BK / 16; ++c) {
        const u32x2 lo = lds_read_tr16(vs + 16 * c * ROWB + offV[db]);
        const u32x2 hi = lds_read_tr16(vs + (16 * c + 8) * ROWB + offV[db]);
        const u32x4 av = {lo[0], lo[1], hi[0], hi[1]};
        acc[db] = mfma32x32x16(as_bf16x8(av), pf[c], acc[db]);
      }
    }
  };

  // Tile t lives in stage t % NS.  Before computing tile t: its loads have
  // landed for every wave.  After: wait for tile t+1 (tiles t+2.. may still
  // load), one barrier (every wave is done with stage t % NS and has tile
  // t+1), then tile t+NS is loaded into stage t % NS.
  issue(0, st0);
  wait_vmcnt<NL>();  // q's loads (issued before tile 0's) have landed
  issue(1, st1);
  if constexpr (NS > 2) issue(2, st2);
  wait_vmcnt<(NS - 1) * NL>();
  stage_barrier();
  for (int t = 0; t < n_tiles; t += NS) {
    compute(t, st0);
    wait_vmcnt<(NS - 2) * NL>();
    stage_barrier();
    issue(t + NS, st0);
    compute(t + 1, st1);
    wait_vmcnt<(NS - 2) * NL>();
    stage_barrier();
    issue(t + NS + 1, st1);
    if constexpr (NS > 2) {
      compute(t + 2, st2);
      wait_vmcnt<(NS - 2) * NL>();
      stage_barrier();
      issue(t + NS + 2, st2);
    }
  }
  wait_vmcnt<0>();

  const float l_tot = xor32_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row_in) {
    uint16_t* orow = (uint16_t*)a.o + ((size_t)(g.b * a.Lq + g.qi) * a.Hq + g.h) * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        u32x2 pk;
        pk[0] = pack_bf16x2(acc[db][4 * gq] * inv, acc[db][4 * gq + 1] * inv);
        pk[1] = pack_bf16x2(acc[db][4 * gq + 2] * inv, acc[db][4 * gq + 3] * inv);
        *(u32x2*)(orow + db * 32 + 8 * gq + 4 * half) = pk;
      }
    if (a.lse && half == 0)
      a.lse[((size_t)g.b * a.Hq + g.h) * a.Lq + g.qi] =
          l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : INFINITY;
  }
}

int launch_flash_bias_ring(int head_dim, const FlashArgs& a, hipStream_t stream) {
  const long blocks = (long)a.n_qtiles * a.B * a.Hq;
  if (head_dim == 128)
    hipLaunchKernelGGL(flash_fwd_bf16_bias_ring_kernel<128>, dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(flash_fwd_bf16_bias_ring_kernel<64>, dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  return check_launch("pjx_flash_fwd");
}

}  // namespace pjx
