// Definitions shared by the flash-attention forward kernels of
// flash_fwd.hip and flash_bias_ring.hip: the argument block, the per-block
// geometry, the bias loader and the bf16 K/V tile layout.
#pragma once

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
};

constexpr int kBQ = 128;
constexpr int kThreads = 256;

// Per-block geometry shared by both dtype paths.
struct BlockGeom {
  int b, h, hkv, q0, qw, qi;
  int q_hi;     // rows >= q_hi are fully masked (QKVLengthMask / Lq)
  int kv_end;   // keys >= kv_end are masked (KVLenMask, QKVLengthMask, Lk)
  int kv_stop;  // keys the block visits (kv_end, clipped causally)
};

__device__ __forceinline__ BlockGeom block_geom(const FlashArgs& a) {
  BlockGeom g;
  const int BH = a.B * a.Hq;
  const int idx = blockIdx.x;
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
  return g;
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
// bytes, 16-byte chunks XOR-swizzled per row (K: chunk ^ (row & (NC-1)); V:
// chunk ^ f(row) chosen so a transposing read of 4 rows x 32 bytes per 16
// lanes hits distinct banks).
template <int D>
struct Bf16Tile {
  static constexpr int BK = 64;             // keys per tile
  static constexpr int ROWB = D * 2;        // bytes per K/V row
  static constexpr int NC = D / 8;          // 16-byte chunks per row
  static constexpr int TILE_B = BK * ROWB;  // bytes of one K (or V) tile
  static constexpr int STAGE_B = 2 * TILE_B;
  static constexpr int RPI = 64 / NC;       // rows per 1 KiB buffer->LDS load
  static constexpr int NLD = (BK / 4) / RPI;  // loads per wave per tensor per tile
  __device__ static int swz_k(int r) { return r & (NC - 1); }
  __device__ static int swz_v(int r) {
    return D == 128 ? 4 * (r & 3) + 2 * ((r >> 1) & 1) : 4 * ((r >> 1) & 1) + 2 * (r & 1);
  }
};

// Launches the bf16 dense-bias kernel (flash_bias_ring.hip); returns a PJX_*
// status.
int launch_flash_bias_ring(int head_dim, const FlashArgs& a, hipStream_t stream);

}  // namespace pjx
