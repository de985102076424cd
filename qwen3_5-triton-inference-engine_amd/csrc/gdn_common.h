// Device code shared by the Gated DeltaNet kernels (gdn.hip, gdn_block.hip):
// the lane layout of a state block and one delta-rule step, so the fused
// decode block and the standalone recurrence run identical arithmetic.
//
// One wavefront owns 16 value columns of one (sequence, head) with all
// DK = 128 key rows.  Lane = kg + 16 * cg: kg (0..15) picks key rows
// 8kg..8kg+7, cg (0..3) picks columns 4cg..4cg+3 of the wave's 16, so a lane
// holds 8 x 4 fp32 state values and every reduction over the key rows stays
// inside one 16-lane DPP row (no LDS, no barrier per token).
#pragma once

#include "wy_common.h"

namespace wy {
namespace gdn {

constexpr int kDK = 128;      // key rows per state (Qwen3.5 linear attention)
constexpr int kRows = 8;      // key rows per lane
constexpr int kCols = 4;      // value columns per lane
constexpr int kWaveCols = 16; // value columns per wavefront

struct GdnArgs {
  const bf16_t *q, *k, *v;
  int64_t q_t, q_h, q_d, k_t, k_h, k_d, v_t, v_h, v_d;
  const float *beta, *g;
  int64_t beta_t, beta_h, g_t, g_h;
  bf16_t *out;
  int64_t o_t, o_h, o_d;
  float *state;
  int64_t s_b, s_h, s_k, s_v;
  const int32_t *cu_seqlens;  // prefill only
  int heads, dv;
};

template <int kRor>
__device__ __forceinline__ float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + kRor, 0xf, 0xf,
                                                    false));
}
// Sum over each 16-lane row; the rotation butterfly gives every lane of the
// row the same value (each level pairs lanes symmetrically).
__device__ __forceinline__ float sum16(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  return v;
}

// 8 consecutive bf16 (key rows 8kg..8kg+7) as fp32.
template <bool kContig>
__device__ __forceinline__ void load8(const bf16_t *p, int64_t stride, float (&x)[kRows]) {
  if constexpr (kContig) {
    const u32x4_t w = ld16(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = bf16_lo(w[e]);
      x[2 * e + 1] = bf16_hi(w[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < kRows; ++e) x[e] = bf16_to_f32(p[e * stride]);
  }
}
template <bool kContig>
__device__ __forceinline__ void load4(const bf16_t *p, int64_t stride, float (&x)[kCols]) {
  if constexpr (kContig) {
    const u32x2_t w = *reinterpret_cast<const u32x2_t *>(p);
    x[0] = bf16_lo(w[0]);
    x[1] = bf16_hi(w[0]);
    x[2] = bf16_lo(w[1]);
    x[3] = bf16_hi(w[1]);
  } else {
#pragma unroll
    for (int e = 0; e < kCols; ++e) x[e] = bf16_to_f32(p[e * stride]);
  }
}
template <bool kContig>
__device__ __forceinline__ void store4(bf16_t *p, int64_t stride, const float (&x)[kCols]) {
  if constexpr (kContig) {
    *reinterpret_cast<u32x2_t *>(p) = u32x2_t{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
  } else {
#pragma unroll
    for (int e = 0; e < kCols; ++e) p[e * stride] = bf16_t(f32_to_bf16_bits(x[e]));
  }
}

// One token's inputs for one lane (NC value columns).
template <int NC>
struct TokenInT {
  float k[kRows], q[kRows], v[NC];
  float g, beta;
};
using TokenIn = TokenInT<kCols>;

template <bool kContig, int NC = kCols>
__device__ __forceinline__ void load_token(const GdnArgs &a, int64_t t, int h, int kg, int col,
                                           TokenInT<NC> &in) {
  load8<kContig>(a.k + t * a.k_t + h * a.k_h + kg * kRows * a.k_d, a.k_d, in.k);
  load8<kContig>(a.q + t * a.q_t + h * a.q_h + kg * kRows * a.q_d, a.q_d, in.q);
  const bf16_t *vp = a.v + t * a.v_t + h * a.v_h + col * a.v_d;
  if constexpr (NC == kCols)
    load4<kContig>(vp, a.v_d, in.v);
  else
#pragma unroll
    for (int e = 0; e < NC; ++e) in.v[e] = bf16_to_f32(vp[e * a.v_d]);
  in.g = a.g[t * a.g_t + h * a.g_h];
  in.beta = a.beta[t * a.beta_t + h * a.beta_h];
}

// One token's inputs as loaded (bf16 bits, fp32 g / beta), for prefetching:
// the bf16 -> fp32 unpack happens at the step (unpack_token), so the loads of
// later tokens stay in flight while a step runs.  g and beta are read through
// VGPR addresses: vector loads complete in order, so waiting for this token's
// values does not wait for the prefetches issued after them (scalar loads
// return out of order and a wait on one is a wait on all).
template <int NC>
struct TokenRaw {
  u32x4_t k, q;
  uint32_t v[NC == kCols ? 2 : NC];
  float g, beta;
};
typedef const __attribute__((address_space(1))) float gfloat_t;

template <bool kContig, int NC>
__device__ __forceinline__ void load_token_raw(const GdnArgs &a, int64_t t, int h, int kg, int col,
                                               TokenRaw<NC> &r) {
  const bf16_t *kp = a.k + t * a.k_t + h * a.k_h + kg * kRows * a.k_d;
  const bf16_t *qp = a.q + t * a.q_t + h * a.q_h + kg * kRows * a.q_d;
  const bf16_t *vp = a.v + t * a.v_t + h * a.v_h + col * a.v_d;
  if constexpr (kContig) {
    r.k = ld16(kp);
    r.q = ld16(qp);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r.k[e] = uint32_t(kp[2 * e * a.k_d]) | (uint32_t(kp[(2 * e + 1) * a.k_d]) << 16);
      r.q[e] = uint32_t(qp[2 * e * a.q_d]) | (uint32_t(qp[(2 * e + 1) * a.q_d]) << 16);
    }
  }
  if constexpr (NC == kCols) {
    if constexpr (kContig) {
      const u32x2_t w = *reinterpret_cast<const u32x2_t *>(vp);
      r.v[0] = w[0];
      r.v[1] = w[1];
    } else {
      r.v[0] = uint32_t(vp[0]) | (uint32_t(vp[a.v_d]) << 16);
      r.v[1] = uint32_t(vp[2 * a.v_d]) | (uint32_t(vp[3 * a.v_d]) << 16);
    }
  } else {
#pragma unroll
    for (int e = 0; e < NC; ++e) r.v[e] = uint32_t(vp[e * a.v_d]);
  }
  gfloat_t *gp = (gfloat_t *)(a.g + t * a.g_t + h * a.g_h);
  gfloat_t *bp = (gfloat_t *)(a.beta + t * a.beta_t + h * a.beta_h);
  asm volatile("" : "+v"(gp), "+v"(bp));
  r.g = *gp;
  r.beta = *bp;
}

template <int NC>
__device__ __forceinline__ TokenInT<NC> unpack_token(const TokenRaw<NC> &r) {
  TokenInT<NC> in;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    in.k[2 * e] = bf16_lo(r.k[e]);
    in.k[2 * e + 1] = bf16_hi(r.k[e]);
    in.q[2 * e] = bf16_lo(r.q[e]);
    in.q[2 * e + 1] = bf16_hi(r.q[e]);
  }
  if constexpr (NC == kCols) {
    in.v[0] = bf16_lo(r.v[0]);
    in.v[1] = bf16_hi(r.v[0]);
    in.v[2] = bf16_lo(r.v[1]);
    in.v[3] = bf16_hi(r.v[1]);
  } else {
#pragma unroll
    for (int e = 0; e < NC; ++e) in.v[e] = bf16_lo(r.v[e]);
  }
  in.g = r.g;
  in.beta = r.beta;
  return in;
}

// One delta-rule step on the lane's 8 x 4 block of S; returns the lane's 4
// output columns (identical in all 16 lanes of the row).
__device__ __forceinline__ void gdn_step(float (&s)[kRows][kCols], const TokenIn &in,
                                         float (&o)[kCols]) {
  const float e = __expf(in.g);
  float mem[kCols], qs[kCols], qk = 0.f;
#pragma unroll
  for (int j = 0; j < kCols; ++j) {
    mem[j] = 0.f;
    qs[j] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    qk = __fmaf_rn(in.q[i], in.k[i], qk);
#pragma unroll
    for (int j = 0; j < kCols; ++j) {
      s[i][j] = e * s[i][j];
      mem[j] = __fmaf_rn(in.k[i], s[i][j], mem[j]);
      qs[j] = __fmaf_rn(in.q[i], s[i][j], qs[j]);
    }
  }
  qk = sum16(qk);
#pragma unroll
  for (int j = 0; j < kCols; ++j) {
    mem[j] = sum16(mem[j]);
    qs[j] = sum16(qs[j]);
  }
  float delta[kCols];
#pragma unroll
  for (int j = 0; j < kCols; ++j) {
    delta[j] = in.beta * (in.v[j] - mem[j]);
    o[j] = __fmaf_rn(qk, delta[j], qs[j]);
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i)
#pragma unroll
    for (int j = 0; j < kCols; ++j) s[i][j] = __fmaf_rn(in.k[i], delta[j], s[i][j]);
}

// The same step on a lazily decayed state: the true state is c * s.  The
// decay only scales c; the reductions use s and are scaled by c, and the
// rank-1 update adds k (delta / c).  When c drops below 2^-32 it is folded
// into s first (c = 0, a full decay, clears s).  This saves the per-element
// decay multiply of every token (3 instead of 4 VALU ops per state element);
// the values agree with gdn_step to fp32 rounding.
template <int NC = kCols>
__device__ __forceinline__ void gdn_step_scaled(float (&s)[kRows][NC], float &c,
                                                const TokenInT<NC> &in, float (&o)[NC]) {
  c *= __expf(in.g);
  if (c < 0x1p-32f) {  // uniform: c depends on the token only
#pragma unroll
    for (int i = 0; i < kRows; ++i)
#pragma unroll
      for (int j = 0; j < NC; ++j) s[i][j] *= c;
    c = 1.f;
  }
  float mem[NC], qs[NC], qk = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    mem[j] = 0.f;
    qs[j] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    qk = __fmaf_rn(in.q[i], in.k[i], qk);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      mem[j] = __fmaf_rn(in.k[i], s[i][j], mem[j]);
      qs[j] = __fmaf_rn(in.q[i], s[i][j], qs[j]);
    }
  }
  qk = sum16(qk);
  const float inv_c = __builtin_amdgcn_rcpf(c);  // v_rcp_f32 (1 ulp): only scales the update
  float dsc[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const float delta = in.beta * (in.v[j] - c * sum16(mem[j]));
    o[j] = __fmaf_rn(qk, delta, c * sum16(qs[j]));
    dsc[j] = delta * inv_c;
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i)
#pragma unroll
    for (int j = 0; j < NC; ++j) s[i][j] = __fmaf_rn(in.k[i], dsc[j], s[i][j]);
}

}  // namespace gdn
}  // namespace wy
