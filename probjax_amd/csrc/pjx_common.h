// Shared device helpers for the probjax_amd attention kernels (gfx950 only).
//
// MFMA lane layouts used throughout (checked on the device against a CPU
// matmul):
//   v_mfma_f32_32x32x16_bf16 : A lane l holds A[l%32][8*(l/32)+j], j<8;
//                              B lane l holds B[8*(l/32)+j][l%32];
//                              C reg r of lane l is C[8*(r/4)+4*(l/32)+r%4][l%32].
//   v_mfma_f32_16x16x32_bf16 : A lane l holds A[l%16][8*(l/16)+j];
//                              B lane l holds B[8*(l/16)+j][l%16];
//                              C reg r of lane l is C[4*(l/16)+r][l%16].
//   v_mfma_f32_16x16x16_bf16 : A lane l holds A[l%16][4*(l/16)+j], j<4;
//                              B lane l holds B[4*(l/16)+j][l%16]; C as for 16x16x32.
//   v_mfma_f32_32x32x2f32    : A lane l holds A[l%32][l/32]; B lane l holds
//                              B[l/32][l%32]; C as for 32x32x16.
// The fp16 forms (v_mfma_f32_32x32x16_f16 etc.) have the same layouts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pjx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Finite "minus infinity" for running maxima (log2 units): masked scores are
// -inf, so exp2(-inf - kMaxInit) == 0 while exp2(kMaxInit - kMaxInit) == 1.
constexpr float kMaxInit = -1e30f;

__device__ __forceinline__ f32x16 mfma32x32x2f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Value of lane l^32 combined with lane l, identical in both halves.
__device__ __forceinline__ float xor32_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Value of lane l^16 combined with lane l (16-lane rows swapped pairwise).
__device__ __forceinline__ float xor16_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Two floats -> packed bf16 pair (round to nearest even; v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 p;
  p[0] = (__bf16)lo;
  p[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, p);
}

// Select 16-bit halves of two dwords: lo halves (sel 0) or hi halves (sel 1)
// of a and b packed as {a_half, b_half}.
__device__ __forceinline__ uint32_t pack_lo_halves(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi_halves(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

template <typename T>
__device__ __forceinline__ T ldg_or_zero(const T* p, bool ok) {
  if (ok) return *p;
  T z;
  __builtin_memset(&z, 0, sizeof(T));
  return z;
}

}  // namespace pjx

namespace pjx {

// ---------------------------------------------------------------------------
// Buffer resources, buffer -> LDS loads and the transposing LDS read (gfx950).
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef uint16_t b16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Raw buffer over [base, base + bytes): loads at offsets >= bytes return 0.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // The descriptor lives in scalar registers, so base and bytes must be the
  // same in every lane; reading them from the first lane states that to the
  // compiler.  A value it cannot prove uniform (e.g. a clamp it computes as
  // v_med3) would otherwise wrap every load in a per-lane waterfall loop.
  const uint64_t p = (uint64_t)base;
  const uint64_t pu = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32)) << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  return __builtin_amdgcn_make_buffer_rsrc((void*)pu, (short)0, __builtin_amdgcn_readfirstlane((int)bytes),
                                           0x00020000);
}

// Each lane loads 16 bytes at voffset; lane l's bytes land at lds_wave + 16*l
// (lds_wave must be the same for every lane of the wave).
__device__ __forceinline__ void buffer_load_lds16(rsrc_t r, void* lds_wave, uint32_t voffset,
                                                  uint32_t soffset = 0) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_wave, 16,
                                           voffset, soffset, 0, 0);
}

// buffer_load_lds16 with the non-temporal hint (data read once per call).
__device__ __forceinline__ void buffer_load_lds16_nt(rsrc_t r, void* lds_wave, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_wave, 16,
                                           voffset, 0, 0, 2 /* nt */);
}

// Each lane loads 4 bytes at voffset; lane l's bytes land at lds_wave + 4*l.
__device__ __forceinline__ void buffer_load_lds4(rsrc_t r, void* lds_wave, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_wave, 4,
                                           voffset, 0, 0, 0);
}

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element
// i%4 of the 8-byte words addressed by lanes i/4, i/4+4, i/4+8, i/4+12 (in
// that order).  Pointing lane s at row (s/4), 16-bit columns 4*(s%4)..+3 of a
// row-major tile hands lane i column i of 4 consecutive rows: a transposed
// 4 x 16 block.  (Lane layout measured on MI355X.)
__device__ __forceinline__ u32x2 lds_read_tr16(const void* p) {
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
  return __builtin_bit_cast(u32x2, v);
}

__device__ __forceinline__ bool wave_any(bool pred) { return __builtin_amdgcn_ballot_w64(pred) != 0; }

// Issue order for a basic block whose N MFMAs each take an operand read from
// LDS just before it (R reads per MFMA): the first PF MFMAs' reads, then each
// MFMA followed by the reads of the one PF places later, so PF MFMAs' reads
// are in flight under the MFMAs.  At high register counts the scheduler
// otherwise issues each read right before its MFMA and waits for it.  Expand
// after the loop that forms the MFMAs, in the same basic block.  (A macro:
// written as an inline function, the same sequence was not applied to the
// latent forward kernel's block.)
#define PJX_SCHED_LDS_READS_AHEAD(N, PF, R)                                \
  do {                                                                     \
    static_assert((N) > (PF) && (PF) > 0, "prefetch depth");               \
    __builtin_amdgcn_sched_group_barrier(0x100, (R) * (PF), 0); /* DS */   \
    _Pragma("unroll") for (int i_ = 0; i_ < (N) - (PF); ++i_) {            \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); /* MFMA */       \
      __builtin_amdgcn_sched_group_barrier(0x100, (R), 0);                 \
    }                                                                      \
    __builtin_amdgcn_sched_group_barrier(0x008, (PF), 0);                  \
  } while (0)

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14.
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier for the buffer->LDS ring.  __syncthreads() carries a
// workgroup release fence, which waits for every outstanding vector memory
// operation of the wave -- including the next tile's loads, still in flight by
// design.  Here the waits are explicit instead: this wave's LDS reads are
// complete (lgkmcnt(0)) and the caller has waited for the loads whose data
// the other waves will read (vmcnt); the wavefront-scope fences only keep the
// compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Lazy softmax rescale: the running max used for exponentiation is raised
// only when a row's new max exceeds it by more than this (log2 units), so P
// stays <= 2^kRescaleLog2 and the O rescale runs on few tiles.
constexpr float kRescaleLog2 = 8.0f;

// ---------------------------------------------------------------------------
// The two 16-bit element formats of the MFMA kernels.  bf16 and fp16 operands
// have the same lane layouts for every instruction used here and the same
// byte layout in memory and LDS, so a kernel templated on the format differs
// only in the MFMA opcodes and the float <-> 16-bit conversions (both round to
// nearest even).  P <= 2^kRescaleLog2 keeps the unnormalised probabilities
// well inside fp16's range.
// ---------------------------------------------------------------------------
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

struct Bf16Fmt {
  typedef bf16x8 v8;
  static constexpr bool kF16 = false;
  __device__ static v8 as8(u32x4 v) { return __builtin_bit_cast(v8, v); }
  __device__ static f32x16 mma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static f32x4 mma16(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static f32x4 mma16k16(s16x4 a, s16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
  __device__ static uint16_t bits(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
  // the element in the low / high 16 bits of a dword, as float
  __device__ static float lo(uint32_t x) { return __uint_as_float(x << 16); }
  __device__ static float hi(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }
};

struct F16Fmt {
  typedef f16x8 v8;
  static constexpr bool kF16 = true;
  __device__ static v8 as8(u32x4 v) { return __builtin_bit_cast(v8, v); }
  __device__ static f32x16 mma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static f32x4 mma16(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static f32x4 mma16k16(s16x4 a, s16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b),
                                                 c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float lo, float hi) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    f16x2 p;
    p[0] = (_Float16)lo;
    p[1] = (_Float16)hi;
    return __builtin_bit_cast(uint32_t, p);
  }
  __device__ static uint16_t bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
  __device__ static float lo(uint32_t x) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(x & 0xffffu)); }
  __device__ static float hi(uint32_t x) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(x >> 16)); }
};

}  // namespace pjx
