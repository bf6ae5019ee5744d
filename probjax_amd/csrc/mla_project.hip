// Up-projection of the shared latent for materialised latent attention:
//
//   k[b, s, h, d] = sum_r cache[b, s, r] * wk[h, d, r]   (d < qk_dim, else 0)
//   v[b, s, h, d] = sum_r cache[b, s, r] * wv[h, d, r]   (d < v_dim,  else 0)
//
// for d < width, fp32 accumulation rounded to the storage dtype.  This is
// `_materialize_kv` (probjax/nn/pallas_kernels/kernels/latent_attention.py:
// 396-410) with the zero head-dim padding of `_materialized_mla` (:413-468,
// `_pad_head_dim`) written by the same pass, so that the flash kernels take K
// and V directly.  The reference's Triton kernel forms these tiles inside its
// KV loop (:132-177) once per query block; here they are formed once per call:
// for L query rows that saves (L / 128 - 1) recomputations of the whole
// projection, and K/V of a full prefill fit HBM many times over.
//
// As a GEMM: out[m, n] = sum_r C[m, r] W[n, r] with m = b*S + s over the
// latent rows and n = h*width + d over the output channels; both operands
// have the rank contiguous (the "NT" form of Q K^T).  One launch covers K
// (grid.y < ny) and V (grid.y >= ny).
//
// bf16 / fp16 (one kernel template over the 16-bit format): 128 x 128 output tiles, 4 waves of 64 x 64 (2 x 2 MFMA 32x32x16
// blocks).  Ranks that are a multiple of 8 stream chunks of 32 rank entries
// straight from HBM into a 2-stage LDS ring (buffer -> LDS loads, the next
// chunk in flight while the current one is multiplied, one barrier per
// chunk); other ranks stage chunks of 64 through registers with element
// loads.
// fp32: 64 x 64 tiles of plain FMA, 4 x 4 per thread (no roundings).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "pjx_common.h"
#include "pjx_internal.h"

namespace pjx {
namespace {

struct ProjArgs {
  const void* cache;  // [M, R]
  const void* w[2];   // [H, dim, R]
  void* out[2];       // [M, H * width]
  int64_t M;          // latent rows B * S
  int H, R, width;
  int dim[2];         // qk_dim, v_dim
  int ny;             // column tiles per output
};

// ---------------------------------------------------------------------------
// bf16
// ---------------------------------------------------------------------------
constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kPitch = kBK * 2 + 16;  // LDS bytes per staged row (16 B pad: fewer bank conflicts)
constexpr int kChunks = kBK / 8;      // 16-byte chunks per staged row
constexpr int kPerThread = kBM * kChunks / 256;

__device__ __forceinline__ u32x4 load_chunk_bf16(const uint16_t* row, int r0, int R, bool vec) {
  // 8 consecutive rank entries r0 .. r0+7 of one row (0 past R / for a null row)
  if (!row) return u32x4{0u, 0u, 0u, 0u};
  if (vec) {
    if (r0 + 8 <= R) return *(const u32x4*)(row + r0);
    return u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t h[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = (r0 + j < R) ? row[r0 + j] : 0u;
  return u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
}

// Ranks that are not a multiple of 8: register-staged chunks, element loads.
template <typename E>
__global__ __launch_bounds__(256, 2) void mla_project_bf16_ragged_kernel(ProjArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * kBM * kPitch];
  unsigned char* As = lds;
  unsigned char* Bs = lds + kBM * kPitch;

  const int which = blockIdx.y >= (unsigned)a.ny ? 1 : 0;
  const int n0 = (blockIdx.y - which * a.ny) * kBN;
  const int64_t m0 = (int64_t)blockIdx.x * kBM;
  const int ncols = a.H * a.width;
  const int dim = a.dim[which];
  const uint16_t* C = (const uint16_t*)a.cache;
  const uint16_t* W = (const uint16_t*)a.w[which];
  const bool vec = (a.R & 7) == 0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // Source rows of this thread's staged chunks (null: zero row).
  const uint16_t* arow[kPerThread];
  const uint16_t* brow[kPerThread];
  int part[kPerThread];
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int c = tid + i * 256;
    const int row = c / kChunks;
    part[i] = c % kChunks;
    const int64_t m = m0 + row;
    arow[i] = m < a.M ? C + m * a.R : nullptr;
    const int n = n0 + row;
    const int h = n / a.width, d = n - h * a.width;
    brow[i] = (n < ncols && d < dim) ? W + ((int64_t)h * dim + d) * a.R : nullptr;
  }

  u32x4 ra[kPerThread], rb[kPerThread];
  auto load = [&](int r0) {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      ra[i] = load_chunk_bf16(arow[i], r0 + 8 * part[i], a.R, vec);
      rb[i] = load_chunk_bf16(brow[i], r0 + 8 * part[i], a.R, vec);
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
  const int frag = (lane & 31) * kPitch + (lane >> 5) * 16;
  const int nk = (a.R + kBK - 1) / kBK;
  load(0);
  for (int t = 0; t < nk; ++t) {
    __syncthreads();  // the previous chunk's reads are done
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int c = tid + i * 256;
      const int off = (c / kChunks) * kPitch + (c % kChunks) * 16;
      *(u32x4*)(As + off) = ra[i];
      *(u32x4*)(Bs + off) = rb[i];
    }
    __syncthreads();
    if (t + 1 < nk) load((t + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      typename E::v8 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = E::as8(*(const u32x4*)(As + (wr + 32 * i) * kPitch + frag + ks * 32));
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = E::as8(*(const u32x4*)(Bs + (wc + 32 * j) * kPitch + frag + ks * 32));
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = E::mma32(af[i], bf[j], acc[i][j]);
    }
  }

  // Register r of block (i, j): row wr + 32i + 8(r/4) + 4(lane/32) + r%4,
  // column wc + 32j + lane%32.
  uint16_t* O = (uint16_t*)a.out[which];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wc + 32 * j + (lane & 31);
      if (n >= ncols) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wr + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < a.M) O[m * ncols + n] = E::bits(acc[i][j][r]);
      }
    }
}

// Ranks that are a multiple of 8: buffer -> LDS ring.  A staged row holds
// 32 rank entries (64 bytes, 4 chunks of 16); chunk c of row r sits in slot
// c ^ ((r / 4) % 4), so the 16 rows one pass of an MFMA operand read touches
// cover the 64 banks once.  One buffer -> LDS load moves 16 rows (64 lanes x
// 16 bytes).  34 KiB of LDS per workgroup: 4 workgroups per CU.
constexpr int kRK = 32;                // rank entries per ring chunk
constexpr int kRowB = kRK * 2;
constexpr int kTileB = kBM * kRowB;    // one operand's chunk: 8 KiB
constexpr int kStageB = 2 * kTileB;    // A and B
constexpr uint32_t kOff = 0x80000000u;  // a buffer offset past every range: loads 0
constexpr int kOutPitch = kBN * 2 + 16;  // LDS bytes per output row in the epilogue
constexpr int kLdsB = 2 * kStageB > kBM * kOutPitch ? 2 * kStageB : kBM * kOutPitch;

template <typename E>
__global__ __launch_bounds__(256, 2) void mla_project_bf16_kernel(ProjArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsB];
  const int which = blockIdx.y >= (unsigned)a.ny ? 1 : 0;
  const int n0 = (blockIdx.y - which * a.ny) * kBN;
  const int64_t m0 = (int64_t)blockIdx.x * kBM;
  const int ncols = a.H * a.width;
  const int dim = a.dim[which];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // (readfirstlane: the descriptor fields must be wave-uniform scalars)
  const uint32_t abytes = __builtin_amdgcn_readfirstlane((uint32_t)(min<int64_t>(kBM, a.M - m0) * a.R * 2));
  const uint32_t bbytes = __builtin_amdgcn_readfirstlane((uint32_t)((int64_t)a.H * dim * a.R * 2));
  const rsrc_t ra = make_rsrc((const uint16_t*)a.cache + m0 * a.R, abytes);
  const rsrc_t rb = make_rsrc(a.w[which], bbytes);

  // This lane's rows in its wave's 2 loads per operand: wave*32 + 16*i +
  // lane/4; it fetches logical chunk (lane%4) ^ ((row/4)%4) of each.
  const int lrow = lane >> 2;
  const int lchunk = (lane & 3) ^ ((lrow >> 2) & 3);  // (row/4)%4 == (lrow/4)%4
  uint32_t aoff[2], boff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = wave * 32 + 16 * i + lrow;
    aoff[i] = (uint32_t)(row * a.R + 8 * lchunk) * 2u;
    const int n = n0 + row;
    const int h = n / a.width, d = n - h * a.width;
    boff[i] = (n < ncols && d < dim) ? (uint32_t)(((int64_t)h * dim + d) * a.R + 8 * lchunk) * 2u : kOff;
  }
  auto issue = [&](int t, int stage) {
    const int k0 = t * kRK;
    const bool in = k0 + 8 * lchunk < a.R;  // chunks past the rank load 0
    unsigned char* base = lds + stage * kStageB + wave * 32 * kRowB;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      buffer_load_lds16(ra, base + 16 * i * kRowB, in ? aoff[i] + 2u * k0 : kOff);
      buffer_load_lds16(rb, base + kTileB + 16 * i * kRowB, (in && boff[i] != kOff) ? boff[i] + 2u * k0 : kOff);
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
  // operand reads: row (lane % 32) of a 32-row block, logical chunk 2*ks + lane/32
  const int rrow = lane & 31, rsw = (rrow >> 2) & 3;
  const int nk = (a.R + kRK - 1) / kRK;
  issue(0, 0);
  for (int t = 0; t < nk; ++t) {
    wait_vmcnt<0>();
    stage_barrier();  // chunk t landed for every wave; every wave is done with chunk t-1
    if (t + 1 < nk) issue(t + 1, (t + 1) & 1);
    const unsigned char* As = lds + (t & 1) * kStageB;
    const unsigned char* Bs = As + kTileB;
#pragma unroll
    for (int ks = 0; ks < kRK / 16; ++ks) {
      const int slot = 16 * ((2 * ks + (lane >> 5)) ^ rsw);
      typename E::v8 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = E::as8(*(const u32x4*)(As + (wr + 32 * i + rrow) * kRowB + slot));
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = E::as8(*(const u32x4*)(Bs + (wc + 32 * j + rrow) * kRowB + slot));
      // W as the MFMA's first operand: the result is out^T, so each lane ends
      // with 4 consecutive output columns of one row per register group
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = E::mma32(bf[j], af[i], acc[i][j]);
    }
  }

  // The 128 x 128 bf16 tile goes through LDS so that the HBM stores are
  // whole 256-byte rows.  Register r of block (i, j): row wr + 32i + lane%32,
  // columns wc + 32j + 8(r/4) + 4(lane/32) + r%4 (4 consecutive per group).
  stage_barrier();  // every wave is done with the ring
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x16& c = acc[i][j];
        const int row = wr + 32 * i + (lane & 31), col = wc + 32 * j + 8 * g + 4 * (lane >> 5);
        *(u32x2*)(lds + row * kOutPitch + col * 2) =
            u32x2{E::pack2(c[4 * g], c[4 * g + 1]), E::pack2(c[4 * g + 2], c[4 * g + 3])};
      }
  stage_barrier();
  uint16_t* O = (uint16_t*)a.out[which];
  const bool vec = (ncols & 7) == 0;
#pragma unroll
  for (int q = 0; q < kBM * kBN / 8 / 256; ++q) {
    const int idx = tid + 256 * q;
    const int row = idx / (kBN / 8), c8 = 8 * (idx % (kBN / 8));
    const int64_t m = m0 + row;
    const int n = n0 + c8;
    if (m >= a.M || n >= ncols) continue;
    const u32x4 v = *(const u32x4*)(lds + row * kOutPitch + c8 * 2);
    uint16_t* dst = O + m * ncols + n;
    if (vec) {
      *(u32x4*)dst = v;
    } else {
      const uint32_t w[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < ncols) dst[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// ---------------------------------------------------------------------------
// fp32
// ---------------------------------------------------------------------------
constexpr int kFM = 64, kFN = 64, kFK = 16;

__global__ __launch_bounds__(256) void mla_project_f32_kernel(ProjArgs a) {
  __shared__ float As[kFK][kFM + 4];
  __shared__ float Bs[kFK][kFN + 4];
  const int which = blockIdx.y >= (unsigned)a.ny ? 1 : 0;
  const int n0 = (blockIdx.y - which * a.ny) * kFN;
  const int64_t m0 = (int64_t)blockIdx.x * kFM;
  const int ncols = a.H * a.width;
  const int dim = a.dim[which];
  const float* C = (const float*)a.cache;
  const float* W = (const float*)a.w[which];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;

  // staging: row tid/4, rank entries 4*(tid%4) .. +3 of the chunk
  const int srow = tid >> 2, sk = 4 * (tid & 3);
  const int64_t m = m0 + srow;
  const float* arow = m < a.M ? C + m * a.R : nullptr;
  const int n = n0 + srow;
  const int h = n / a.width, d = n - h * a.width;
  const float* brow = (n < ncols && d < dim) ? W + ((int64_t)h * dim + d) * a.R : nullptr;

  float acc[4][4] = {};
  for (int r0 = 0; r0 < a.R; r0 += kFK) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = r0 + sk + j;
      As[sk + j][srow] = (arow && r < a.R) ? arow[r] : 0.f;
      Bs[sk + j][srow] = (brow && r < a.R) ? brow[r] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kFK; ++k) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[k][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[k][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
  float* O = (float*)a.out[which];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t mo = m0 + ty * 4 + i;
    if (mo >= a.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int no = n0 + tx * 4 + j;
      if (no < ncols) O[mo * ncols + no] = acc[i][j];
    }
  }
}

}  // namespace
}  // namespace pjx

using namespace pjx;

extern "C" int pjx_mla_project(int dtype, const void* cache, const void* wk, const void* wv, void* k,
                               void* v, int64_t batch, int64_t kv_len, int64_t heads, int64_t rank,
                               int64_t qk_dim, int64_t v_dim, int64_t width, void* stream) {
  clear_error();
  if (dtype != PJX_DTYPE_BF16 && dtype != PJX_DTYPE_F16 && dtype != PJX_DTYPE_F32)
    return fail(PJX_ERR_INVALID, "pjx_mla_project: dtype must be bf16, f16 or f32");
  if (batch < 0 || kv_len < 0 || heads <= 0 || rank <= 0)
    return fail(PJX_ERR_INVALID, "pjx_mla_project: bad sizes");
  if (width <= 0 || qk_dim <= 0 || v_dim <= 0 || qk_dim > width || v_dim > width)
    return fail(PJX_ERR_INVALID, "pjx_mla_project: need 1 <= qk_dim, v_dim <= width");
  if (rank > (1 << 20) || heads * width > (1 << 20) || batch * kv_len > ((int64_t)1 << 34))
    return fail(PJX_ERR_INVALID, "pjx_mla_project: sizes out of range");
  const int64_t M = batch * kv_len;
  if (M == 0) return PJX_OK;
  if (!cache || !wk || !wv || !k || !v) return fail(PJX_ERR_INVALID, "pjx_mla_project: null pointer");
  ProjArgs a = {};
  a.cache = cache;
  a.w[0] = wk;
  a.w[1] = wv;
  a.out[0] = k;
  a.out[1] = v;
  a.M = M;
  a.H = (int)heads;
  a.R = (int)rank;
  a.width = (int)width;
  a.dim[0] = (int)qk_dim;
  a.dim[1] = (int)v_dim;
  const int ncols = a.H * a.width;
  hipStream_t s = (hipStream_t)stream;
  if (dtype != PJX_DTYPE_F32) {
    a.ny = (ncols + kBN - 1) / kBN;
    const int64_t gx = (M + kBM - 1) / kBM;
    if (gx > 0x7fffffff) return fail(PJX_ERR_INVALID, "pjx_mla_project: sizes out of range");
    // the ring's buffer offsets are 32-bit: 128 latent rows and each weight tensor
    const bool ring = (rank & 7) == 0 && 128 * rank * 2 < ((int64_t)1 << 31) &&
                      heads * std::max(qk_dim, v_dim) * rank * 2 < ((int64_t)1 << 31);
    const dim3 grid((unsigned)gx, 2 * a.ny);
    if (dtype == PJX_DTYPE_F16) {
      if (ring)
        launch_kernel<mla_project_bf16_kernel<F16Fmt>>(grid, dim3(256), 0, s, a);
      else
        launch_kernel<mla_project_bf16_ragged_kernel<F16Fmt>>(grid, dim3(256), 0, s, a);
    } else if (ring) {
      launch_kernel<mla_project_bf16_kernel<Bf16Fmt>>(grid, dim3(256), 0, s, a);
    } else {
      launch_kernel<mla_project_bf16_ragged_kernel<Bf16Fmt>>(grid, dim3(256), 0, s, a);
    }
  } else {
    a.ny = (ncols + kFN - 1) / kFN;
    const int64_t gx = (M + kFM - 1) / kFM;
    if (gx > 0x7fffffff) return fail(PJX_ERR_INVALID, "pjx_mla_project: sizes out of range");
    launch_kernel<mla_project_f32_kernel>(dim3((unsigned)gx, 2 * a.ny), dim3(256), 0, s, a);
  }
  return check_launch("pjx_mla_project");
}
