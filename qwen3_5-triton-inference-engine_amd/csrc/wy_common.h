// Shared device/host helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wy_attn.h"

namespace wy {

typedef uint16_t bf16_t;  // raw bfloat16 bits

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kPage = WY_PAGE_SIZE;
constexpr int kMaxSplits = WY_MAX_SPLITS;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(bf16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// fp32 -> bf16, round to nearest even; NaN stays NaN (quiet bit set).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
// Two floats -> packed bf16 pair (lo in bits 0..15), round to nearest even:
// one v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
// Round a float to the nearest bf16 value and return it as float.
__device__ __forceinline__ float round_bf16(float f) {
  return __uint_as_float(pack_bf16x2(f, 0.f) << 16);
}

__device__ __forceinline__ u32x4_t ld16(const void *p) {
  return *reinterpret_cast<const u32x4_t *>(p);
}
__device__ __forceinline__ void st16(void *p, u32x4_t v) {
  *reinterpret_cast<u32x4_t *>(p) = v;
}
// Non-temporal 16-byte store (global_store ... nt): for bulk outputs that
// this launch does not read back, so they stream out while the kernel runs
// rather than sit dirty in L2 until the end-of-kernel writeback.
__device__ __forceinline__ void st16_nt(void *p, u32x4_t v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t *>(p));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ---- shared by the standalone RMSNorm / RoPE kernels and the fused decode
// block, so that the fused path is bit-identical to the op-by-op path ------

// out1 = x1*cos - x2*sin, out2 = x1*sin + x2*cos, each product rounded on its
// own (no fused multiply-add), matching the fp32 formula of
// partial_rope.py:97-98.
__device__ __forceinline__ void rope_rotate(float x1, float x2, float c, float s, float &o1,
                                            float &o2) {
  // Plain operators under contract(off): the _rn intrinsics come from the
  // device library with contraction allowed, and after inlining the compiler
  // fused one of the products into the add -- a different one depending on
  // the calling kernel's schedule, so kernels rotating the same values
  // (standalone partial RoPE, K/V fill, prefill and decode blocks) could
  // round apart.
#pragma clang fp contract(off)
  o1 = x1 * c - x2 * s;
  o2 = x1 * s + x2 * c;
}
// angle = float(pos) * inv_freq[j] in fp32 (partial_rope.py:74-75).
__device__ __forceinline__ void rope_sincos(float pos, float inv_freq_j, float &s, float &c) {
  sincosf(__fmul_rn(pos, inv_freq_j), &s, &c);
}

// Position id as float (int32 or int64 tensor).
__device__ __forceinline__ float load_pos(const void *pos, int64_t off, bool is64) {
  return is64 ? float(static_cast<const int64_t *>(pos)[off])
              : float(static_cast<const int32_t *>(pos)[off]);
}
// sigmoid(g) in fp32 as the gate pack computes it (attention_gate_pack.py:56).
__device__ __forceinline__ float gate_sigmoid(float g) { return 1.0f / (1.0f + __expf(-g)); }

// RMSNorm of one row held by a group of 32 consecutive lanes, lane l holding
// 8 consecutive elements of each 256-element block k (elements 8(32k+l) ..).
// The sum of squares runs over the lane's elements in order, then an xor
// tree over the 32 lanes; rsigma = rsqrt(sum/D + eps).  y = x*rsigma*(1+w)
// in fp32 (qwen_rmsnorm.py:69-73).
// Sum of squares of 8 bf16 elements (one 16-byte chunk) into ss, in element
// order, one fused multiply-add each.
__device__ __forceinline__ float rms_acc8(u32x4_t xw, float ss) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    ss = __fmaf_rn(bf16_lo(xw[e]), bf16_lo(xw[e]), ss);
    ss = __fmaf_rn(bf16_hi(xw[e]), bf16_hi(xw[e]), ss);
  }
  return ss;
}
__device__ __forceinline__ float rms_rsigma(float sumsq_lane, int d_model, float eps) {
  float s = sumsq_lane;
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) s += __shfl_xor(s, o);
  return rsqrtf(s / float(d_model) + eps);
}
__device__ __forceinline__ float rms_apply(float x, float rsigma, float w) {
  return (x * rsigma) * (1.0f + w);
}

}  // namespace wy

// Host-side helpers shared by the launchers.
namespace wyh {

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? WY_OK : int(e);
}

}  // namespace wyh
