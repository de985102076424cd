// The Gated DeltaNet decode mixer around the recurrence, on gfx950:
//   * depthwise causal conv4 decode (+ SiLU) with its rolling input state
//     (depthwise_causal_conv4_decode.py:86-150, op :152-205),
//   * per-head q/k L2 norm and the beta / g gates (gdn_qk_norm_gates.py:19-115,
//     op :127-201),
//   * gated RMSNorm of the recurrence output (gdn_gated_rmsnorm.py:21-76,
//     op :88-137),
// each as a standalone kernel, and all of them together with the recurrence
// step as one launch per decode step (the runner's _gdn_decode between the
// fused projection and out_proj, engine/runner.py:431-441).  The fused
// launch calls the same device functions with the same reduction shapes as
// the standalone kernels, so it equals the op-by-op sequence bit for bit.
#include "gdn_common.h"

using namespace wy;
using namespace wy::gdn;

namespace {

// acc = x[t-3] w0 + x[t-2] w1 + x[t-1] w2 + x[t] w3 (fp32, in tap order),
// y = acc * sigmoid(acc) rounded to bf16.
__device__ __forceinline__ float conv4_silu_f(float s1, float s2, float s3, float x, float w0,
                                              float w1, float w2, float w3) {
  float acc = s1 * w0;
  acc = __fmaf_rn(s2, w1, acc);
  acc = __fmaf_rn(s3, w2, acc);
  acc = __fmaf_rn(x, w3, acc);
  return acc * (1.0f / (1.0f + __expf(-acc)));
}
__device__ __forceinline__ uint32_t conv4_silu(float s1, float s2, float s3, float x, float w0,
                                               float w1, float w2, float w3) {
  return f32_to_bf16_bits(conv4_silu_f(s1, s2, s3, x, w0, w1, w2, w3));
}

// Sum of one value per thread over a 128-thread row held by two consecutive
// wavefronts (waves 2r, 2r+1): xor butterfly in each wave, then wave 2r's
// part + wave 2r+1's part.  Every thread of the block must call it (it holds
// a barrier); part needs one float per wave.
__device__ __forceinline__ float sum128(float v, float *part) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) part[wave] = v;
  __syncthreads();
  const int w0 = wave & ~1;
  return part[w0] + part[w0 + 1];
}

// softplus(x) = max(x, 0) + log(1 + exp(-|x|)) (gdn_qk_norm_gates.py:90-93)
__device__ __forceinline__ float softplus(float x) {
  return fmaxf(x, 0.f) + __logf(1.0f + __expf(-fabsf(x)));
}
// beta = sigmoid(b); g = -exp(a_log) * softplus(a + dt_bias)
__device__ __forceinline__ void gdn_gates(float a, float b, float a_log, float dt_bias,
                                          float &beta, float &g) {
  beta = 1.0f / (1.0f + __expf(-b));
  g = -__expf(a_log) * softplus(a + dt_bias);
}
// z * sigmoid(z) with the two-sided form of gdn_gated_rmsnorm.py:56-62
__device__ __forceinline__ float silu_gate(float z) {
  const float e = __expf(-fabsf(z));
  const float sg = z >= 0.f ? 1.0f / (1.0f + e) : e / (1.0f + e);
  return z * sg;
}

// ---- standalone kernels ------------------------------------------------------

// conv4 decode: one thread per (sequence, channel); state [B, 4, C] with the
// channel innermost, weight [4, C].
__global__ __launch_bounds__(256) void conv4_decode_kernel(
    const bf16_t *__restrict__ x, int64_t x_b, int64_t x_c, bf16_t *__restrict__ state,
    int64_t st_b, int64_t st_k, const bf16_t *__restrict__ w, int64_t w_k,
    bf16_t *__restrict__ out, int64_t o_b, int64_t o_c, int C) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (c >= C) return;
  bf16_t *sp = state + b * st_b + c;
  const bf16_t s1 = sp[st_k], s2 = sp[2 * st_k], s3 = sp[3 * st_k];
  const bf16_t xv = x[b * x_b + c * x_c];
  const uint32_t y = conv4_silu(bf16_to_f32(s1), bf16_to_f32(s2), bf16_to_f32(s3),
                                bf16_to_f32(xv), bf16_to_f32(w[c]), bf16_to_f32(w[w_k + c]),
                                bf16_to_f32(w[2 * w_k + c]), bf16_to_f32(w[3 * w_k + c]));
  sp[0] = s1;
  sp[st_k] = s2;
  sp[2 * st_k] = s3;
  sp[3 * st_k] = xv;
  out[b * o_b + c * o_c] = bf16_t(y);
}

struct QkNormArgs {
  const bf16_t *q, *k, *a, *b, *dt_bias;
  const float *a_log;
  int64_t q_t, q_h, q_d, k_t, k_h, k_d, a_t, a_h, b_t, b_h;
  bf16_t *qn, *kn;
  float *beta, *g;
  int64_t qn_t, qn_h, kn_t, kn_h;  // contiguous rows
  int heads;
  float q_scale;
};

// One 256-thread block per (token, head): threads 0..127 normalise q's
// elements, 128..255 k's; thread 0 writes beta and g.
__global__ __launch_bounds__(256) void gdn_qk_norm_gates_kernel(const QkNormArgs p) {
  __shared__ float part[4];
  const int th = blockIdx.x;
  const int t = th / p.heads, h = th - t * p.heads;
  const int c = threadIdx.x & 127;
  const bool is_k = threadIdx.x >= 128;
  const float x = bf16_to_f32(is_k ? p.k[t * p.k_t + h * p.k_h + c * p.k_d]
                                   : p.q[t * p.q_t + h * p.q_h + c * p.q_d]);
  const float ss = sum128(x * x, part);
  const float r = rsqrtf(ss + 1e-6f);
  if (is_k)
    p.kn[t * p.kn_t + h * p.kn_h + c] = bf16_t(f32_to_bf16_bits(x * r));
  else
    p.qn[t * p.qn_t + h * p.qn_h + c] = bf16_t(f32_to_bf16_bits((x * r) * p.q_scale));
  if (threadIdx.x == 0) {
    float beta, g;
    gdn_gates(bf16_to_f32(p.a[t * p.a_t + h * p.a_h]), bf16_to_f32(p.b[t * p.b_t + h * p.b_h]),
              p.a_log[h], bf16_to_f32(p.dt_bias[h]), beta, g);
    p.beta[th] = beta;
    p.g[th] = g;
  }
}

// Gated RMSNorm: one 128-thread block per (token, head), D = 128.
__global__ __launch_bounds__(128) void gdn_gated_rmsnorm_kernel(
    const bf16_t *__restrict__ x, int64_t x_t, int64_t x_h, int64_t x_d,
    const bf16_t *__restrict__ z, int64_t z_t, int64_t z_h, int64_t z_d,
    const float *__restrict__ w, bf16_t *__restrict__ out, int heads) {
  __shared__ float part[2];
  const int th = blockIdx.x;
  const int t = th / heads, h = th - t * heads;
  const int c = threadIdx.x;
  const float xv = bf16_to_f32(x[t * x_t + h * x_h + c * x_d]);
  const float zv = bf16_to_f32(z[t * z_t + h * z_h + c * z_d]);
  const float ss = sum128(xv * xv, part);
  const float inv = rsqrtf(ss / float(kDK) + 1e-6f);
  out[int64_t(th) * kDK + c] = bf16_t(f32_to_bf16_bits(((xv * inv) * w[c]) * silu_gate(zv)));
}

// conv4 prefill (+ SiLU) over a packed batch: one thread per channel walks
// kConvRun consecutive tokens with the 4-tap window in registers, so each
// input row is read once per run (plus 3 rows of halo).  Token t's taps
// below seq_start[t] read as zero (no look-back across sequences).  Same
// arithmetic as the decode step (conv4_silu), so prefill and decode agree bit
// for bit on the same window.
constexpr int kConvRun = 16;
// Row counts from which the norm ops take the row-vectorised kernels (the
// decode sizes keep one block per row, the same reduction either way).
constexpr int kVecRows = 256;

__global__ __launch_bounds__(256) void conv4_prefill_kernel(
    const bf16_t *__restrict__ x, int64_t x_t, int64_t x_c, const bf16_t *__restrict__ w,
    int64_t w_c, int64_t w_k, bf16_t *__restrict__ out, int64_t o_t, int64_t o_c,
    const int32_t *__restrict__ seq_start, int T, int C) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int t0 = blockIdx.y * kConvRun;
  if (c >= C) return;
  const float w0 = bf16_to_f32(w[c * w_c]), w1 = bf16_to_f32(w[c * w_c + w_k]);
  const float w2 = bf16_to_f32(w[c * w_c + 2 * w_k]), w3 = bf16_to_f32(w[c * w_c + 3 * w_k]);
  const bf16_t *xc = x + c * x_c;
  // window: win[j] = x[t0 - 3 + j]
  float win[kConvRun + 3];
#pragma unroll
  for (int j = 0; j < kConvRun + 3; ++j) {
    const int t = t0 - 3 + j;
    win[j] = (t >= 0 && t < T) ? bf16_to_f32(xc[int64_t(t) * x_t]) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < kConvRun; ++i) {
    const int t = t0 + i;
    if (t >= T) break;
    const int lo = seq_start ? seq_start[t] : 0;
    const float a0 = t - 3 >= lo ? win[i] : 0.f;
    const float a1 = t - 2 >= lo ? win[i + 1] : 0.f;
    const float a2 = t - 1 >= lo ? win[i + 2] : 0.f;
    out[int64_t(t) * o_t + c * o_c] = bf16_t(conv4_silu(a0, a1, a2, win[i + 3], w0, w1, w2, w3));
  }
}

// ---- row-vectorised forms for many tokens (prefill) -----------------------
//
// A 16-lane group holds one 128-element row, lane l elements 8l .. 8l + 7
// (one 16-byte load).  row_sum128 adds the 128 values with exactly the
// pairings of sum128 (xor butterfly over element index within each 64-element
// half, offsets 32, 16, 8, 4, 2, 1, then the two halves): offsets 32 / 16 / 8
// are lanes l ^ 4 / 2 / 1, offsets 4 / 2 / 1 are registers j ^ 4 / 2 / 1, the
// halves are lanes l ^ 8.  fp addition is commutative, so every partial sum
// is bit-identical to sum128's and the results match the one-thread-per-
// element kernels (and the fused decode block) bit for bit.
__device__ __forceinline__ float row_sum128(float (&v)[8]) {
#pragma unroll
  for (int o = 4; o > 0; o >>= 1)
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] += __shfl_xor(v[j], o);
  const float a0 = v[0] + v[4], a1 = v[1] + v[5], a2 = v[2] + v[6], a3 = v[3] + v[7];
  const float b0 = a0 + a2, b1 = a1 + a3;
  const float h = b0 + b1;
  return h + __shfl_xor(h, 8);
}

__device__ __forceinline__ void unpack8(const u32x4_t x, float (&f)[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = bf16_lo(x[e]);
    f[2 * e + 1] = bf16_hi(x[e]);
  }
}

// q/k norms and gates: 16 rows per 256-thread block, rows 2i (q) and 2i + 1
// (k) of (token, head) pair 8 blockIdx + i.
__global__ __launch_bounds__(256) void gdn_qk_norm_gates_vec_kernel(const QkNormArgs p,
                                                                    int pairs) {
  const int grp = threadIdx.x >> 4, l = threadIdx.x & 15;
  const int th = blockIdx.x * 8 + (grp >> 1);
  const bool is_k = grp & 1;
  if (th >= pairs) return;   // uniform over the 16-lane group
  const int t = th / p.heads, h = th - t * p.heads;
  const u32x4_t raw = ld16(is_k ? p.k + t * p.k_t + h * p.k_h + 8 * l
                                : p.q + t * p.q_t + h * p.q_h + 8 * l);
  float x[8], sq[8];
  unpack8(raw, x);
#pragma unroll
  for (int j = 0; j < 8; ++j) sq[j] = x[j] * x[j];
  const float r = rsqrtf(row_sum128(sq) + 1e-6f);
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = is_k ? (f32_to_bf16_bits(x[2 * e] * r) | (f32_to_bf16_bits(x[2 * e + 1] * r) << 16))
                : (f32_to_bf16_bits((x[2 * e] * r) * p.q_scale) |
                   (f32_to_bf16_bits((x[2 * e + 1] * r) * p.q_scale) << 16));
  st16(is_k ? p.kn + t * p.kn_t + h * p.kn_h + 8 * l : p.qn + t * p.qn_t + h * p.qn_h + 8 * l, o);
  if (!is_k && l == 0) {
    float beta, g;
    gdn_gates(bf16_to_f32(p.a[t * p.a_t + h * p.a_h]), bf16_to_f32(p.b[t * p.b_t + h * p.b_h]),
              p.a_log[h], bf16_to_f32(p.dt_bias[h]), beta, g);
    p.beta[th] = beta;
    p.g[th] = g;
  }
}

// Gated RMSNorm: 16 (token, head) rows per 256-thread block.
__global__ __launch_bounds__(256) void gdn_gated_rmsnorm_vec_kernel(
    const bf16_t *__restrict__ x, int64_t x_t, int64_t x_h, const bf16_t *__restrict__ z,
    int64_t z_t, int64_t z_h, const float *__restrict__ w, bf16_t *__restrict__ out, int heads,
    int rows) {
  const int l = threadIdx.x & 15;
  const int th = blockIdx.x * 16 + (threadIdx.x >> 4);
  if (th >= rows) return;
  const int t = th / heads, h = th - t * heads;
  float xv[8], zv[8], sq[8];
  unpack8(ld16(x + t * x_t + h * x_h + 8 * l), xv);
  unpack8(ld16(z + t * z_t + h * z_h + 8 * l), zv);
#pragma unroll
  for (int j = 0; j < 8; ++j) sq[j] = xv[j] * xv[j];
  const float inv = rsqrtf(row_sum128(sq) / float(kDK) + 1e-6f);
  const f32x4_t w0 = *reinterpret_cast<const f32x4_t *>(w + 8 * l);
  const f32x4_t w1 = *reinterpret_cast<const f32x4_t *>(w + 8 * l + 4);
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float wa = e < 2 ? w0[2 * e] : w1[2 * e - 4], wb = e < 2 ? w0[2 * e + 1] : w1[2 * e - 3];
    o[e] = f32_to_bf16_bits(((xv[2 * e] * inv) * wa) * silu_gate(zv[2 * e])) |
           (f32_to_bf16_bits(((xv[2 * e + 1] * inv) * wb) * silu_gate(zv[2 * e + 1])) << 16);
  }
  st16(out + int64_t(th) * kDK + 8 * l, o);
}

// conv4 prefill with 8 consecutive channels per thread (16-byte loads and
// stores); per channel the same window and arithmetic as conv4_prefill_kernel.
__global__ __launch_bounds__(256) void conv4_prefill_vec_kernel(
    const bf16_t *__restrict__ x, int64_t x_t, const bf16_t *__restrict__ w, int64_t w_c,
    int64_t w_k, bf16_t *__restrict__ out, int64_t o_t, const int32_t *__restrict__ seq_start,
    int T, int C) {
  const int c0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  const int t0 = blockIdx.y * kConvRun;
  if (c0 >= C) return;
  float wt[4][8];
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int j = 0; j < 8; ++j) wt[k][j] = bf16_to_f32(w[(c0 + j) * w_c + k * w_k]);
  // win[j] = x[t0 - 3 + j, c0 .. c0 + 7].  Rows outside [0, T) read a clamped
  // row instead of branching round the load (loads that only some paths
  // issue make every later wait a wait for all of them): a row before 0 lies
  // before every sequence's start and is masked below, a row from T on only
  // feeds tokens from T on, which are not computed.
  u32x4_t win[kConvRun + 3];
#pragma unroll
  for (int j = 0; j < kConvRun + 3; ++j) {
    const int t = min(max(t0 - 3 + j, 0), T - 1);
    win[j] = ld16(x + int64_t(t) * x_t + c0);
  }
  // each window row is unpacked once into a rolling 4-row float window; the
  // per-row masks for rows before the sequence's start are only evaluated for
  // a token whose window reaches past it (a block-uniform branch); the pair
  // rounding (v_cvt_pk_bf16_f32) equals conv4_silu's for finite values
  float f[4][8];
  unpack8(win[0], f[0]);
  unpack8(win[1], f[1]);
  unpack8(win[2], f[2]);
#pragma unroll
  for (int i = 0; i < kConvRun; ++i) {
    const int t = t0 + i;
    if (t >= T) break;
    unpack8(win[i + 3], f[(i + 3) & 3]);
    const float(&a0)[8] = f[i & 3];
    const float(&a1)[8] = f[(i + 1) & 3];
    const float(&a2)[8] = f[(i + 2) & 3];
    const float(&a3)[8] = f[(i + 3) & 3];
    const int lo = seq_start ? seq_start[t] : 0;
    u32x4_t o;
    if (t - 3 >= lo) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float y[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int j = 2 * e + u;
          y[u] = conv4_silu_f(a0[j], a1[j], a2[j], a3[j], wt[0][j], wt[1][j], wt[2][j],
                              wt[3][j]);
        }
        o[e] = pack_bf16x2(y[0], y[1]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float y[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int j = 2 * e + u;
          y[u] = conv4_silu_f(t - 3 >= lo ? a0[j] : 0.f, t - 2 >= lo ? a1[j] : 0.f,
                              t - 1 >= lo ? a2[j] : 0.f, a3[j], wt[0][j], wt[1][j], wt[2][j],
                              wt[3][j]);
        }
        o[e] = pack_bf16x2(y[0], y[1]);
      }
    }
    st16(out + int64_t(t) * o_t + c0, o);
  }
}

// conv state after a packed prefill: state[b, r, :] = x[end_b - 4 + r, :],
// zero where that row precedes the sequence's start.  Every row is written
// (zeros included), so a reused cache keeps nothing of its previous contents.
__global__ __launch_bounds__(256) void conv_state_pack_kernel(
    const bf16_t *__restrict__ x, int64_t x_t, bf16_t *__restrict__ state, int64_t st_b,
    int64_t st_k, const int32_t *__restrict__ cu_seqlens, int C) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (c >= C) return;
  const int start = cu_seqlens[b], end = cu_seqlens[b + 1];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = end - 4 + r;
    state[b * st_b + r * st_k + c] = t >= start ? x[int64_t(t) * x_t + c] : bf16_t(0);
  }
}

// ---- the fused decode block -----------------------------------------------------

struct BlockArgs {
  const bf16_t *fused;  // [B, 3*H*D + H*D + 2*H]: q|k|v conv inputs, z, a, b
  int64_t f_b;
  bf16_t *conv_state;   // [B, 4, 3*H*D]
  int64_t cs_b, cs_k;
  const bf16_t *conv_w; // [4, 3*H*D]
  int64_t cw_k;
  const float *a_log;
  const bf16_t *dt_bias;
  const float *norm_w;
  float *state;         // [B, H, D, D]
  int64_t s_b, s_h, s_k;
  bf16_t *out;          // [B, H*D]
  int64_t o_b;
  int heads;
  float q_scale;
};

// One 512-thread workgroup per (sequence, head).  The state loads are issued
// first and land while the conv, norms and gates run:
//   1. threads 0..383: conv4 + SiLU of the head's q, k, v channels (state
//      shifted in place); the results go to LDS as bf16 values;
//   2. waves 0-1 / 2-3: q / k L2 norm (sum128, as the standalone kernel);
//   3. every wave: one recurrence step on its 16 value columns (gdn_step);
//   4. waves 0-1: gated RMSNorm of the bf16 step output with z.
__global__ __launch_bounds__(512) void gdn_decode_block_kernel(const BlockArgs p) {
  __shared__ float y_lds[3 * kDK];  // conv outputs (bf16 values): q | k | v
  __shared__ float qk_lds[2 * kDK]; // normalised q | k (bf16 values)
  __shared__ float core[kDK];       // recurrence output (bf16 values)
  __shared__ float part[8];
  const int bh = blockIdx.x;
  const int b = bh / p.heads, h = bh - b * p.heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int kg = lane & 15, cg = lane >> 4;
  const int col = wave * kWaveCols + cg * kCols;
  const int HD = p.heads * kDK;

  float *sp = p.state + b * p.s_b + h * p.s_h + int64_t(kg * kRows) * p.s_k + col;
  float s[kRows][kCols];
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const float4 x = *reinterpret_cast<const float4 *>(sp + i * p.s_k);
    s[i][0] = x.x;
    s[i][1] = x.y;
    s[i][2] = x.z;
    s[i][3] = x.w;
  }
  const bf16_t *frow = p.fused + b * p.f_b;
  float zv = 0.f;
  if (tid < kDK) zv = bf16_to_f32(frow[3 * HD + h * kDK + tid]);

  // 1. conv4 + SiLU
  if (tid < 3 * kDK) {
    const int region = tid >> 7, c = tid & 127;
    const int ch = region * HD + h * kDK + c;
    bf16_t *cs = p.conv_state + b * p.cs_b + ch;
    const bf16_t s1 = cs[p.cs_k], s2 = cs[2 * p.cs_k], s3 = cs[3 * p.cs_k];
    const bf16_t xv = frow[ch];
    const bf16_t *w = p.conv_w + ch;
    const uint32_t y = conv4_silu(bf16_to_f32(s1), bf16_to_f32(s2), bf16_to_f32(s3),
                                  bf16_to_f32(xv), bf16_to_f32(w[0]), bf16_to_f32(w[p.cw_k]),
                                  bf16_to_f32(w[2 * p.cw_k]), bf16_to_f32(w[3 * p.cw_k]));
    cs[0] = s1;
    cs[p.cs_k] = s2;
    cs[2 * p.cs_k] = s3;
    cs[3 * p.cs_k] = xv;
    y_lds[tid] = bf16_to_f32(bf16_t(y));
  }
  float beta, g;
  gdn_gates(bf16_to_f32(frow[4 * HD + h]), bf16_to_f32(frow[4 * HD + p.heads + h]), p.a_log[h],
            bf16_to_f32(p.dt_bias[h]), beta, g);
  __syncthreads();

  // 2. q / k L2 norm: waves 0-1 hold q, waves 2-3 k (threads 256.. add zeros)
  {
    const float x = tid < 2 * kDK ? y_lds[tid] : 0.f;
    const float ss = sum128(x * x, part);
    const float r = rsqrtf(ss + 1e-6f);
    if (tid < kDK)
      qk_lds[tid] = bf16_to_f32(bf16_t(f32_to_bf16_bits((x * r) * p.q_scale)));
    else if (tid < 2 * kDK)
      qk_lds[tid] = bf16_to_f32(bf16_t(f32_to_bf16_bits(x * r)));
  }
  __syncthreads();

  // 3. recurrence step
  TokenIn in;
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    in.q[i] = qk_lds[kg * kRows + i];
    in.k[i] = qk_lds[kDK + kg * kRows + i];
  }
#pragma unroll
  for (int j = 0; j < kCols; ++j) in.v[j] = y_lds[2 * kDK + col + j];
  in.g = g;
  in.beta = beta;
  float o[kCols];
  gdn_step(s, in, o);
#pragma unroll
  for (int i = 0; i < kRows; ++i)
    *reinterpret_cast<float4 *>(sp + i * p.s_k) = make_float4(s[i][0], s[i][1], s[i][2], s[i][3]);
  if (kg == 0) {
#pragma unroll
    for (int j = 0; j < kCols; ++j) core[col + j] = bf16_to_f32(bf16_t(f32_to_bf16_bits(o[j])));
  }
  __syncthreads();

  // 4. gated RMSNorm (waves 0-1; the others add zeros to their own pairs)
  {
    const float x = tid < kDK ? core[tid] : 0.f;
    const float ss = sum128(x * x, part + 0);
    if (tid < kDK) {
      const float inv = rsqrtf(ss / float(kDK) + 1e-6f);
      p.out[b * p.o_b + h * kDK + tid] =
          bf16_t(f32_to_bf16_bits(((x * inv) * p.norm_w[tid]) * silu_gate(zv)));
    }
  }
}

}  // namespace

extern "C" int wy_depthwise_causal_conv4_decode(const void *x, const int64_t *x_strides,
                                                void *state, const int64_t *state_strides,
                                                const void *weight, const int64_t *w_strides,
                                                void *out, const int64_t *out_strides, int batch,
                                                int channels, void *stream) {
  if (!x || !x_strides || !state || !state_strides || !weight || !w_strides || !out ||
      !out_strides)
    return WY_E_NULL;
  if (batch < 0 || channels < 0) return WY_E_SHAPE;
  if (state_strides[2] != 1 || w_strides[1] != 1) return WY_E_LAYOUT;
  if (batch == 0 || channels == 0) return WY_OK;
  const dim3 grid(unsigned((channels + 255) / 256), unsigned(batch));
  conv4_decode_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(x), x_strides[0], x_strides[1], static_cast<bf16_t *>(state),
      state_strides[0], state_strides[1], static_cast<const bf16_t *>(weight), w_strides[0],
      static_cast<bf16_t *>(out), out_strides[0], out_strides[1], channels);
  return wyh::launch_status();
}

extern "C" int wy_gdn_qk_norm_gates(const void *q, const int64_t *q_strides, const void *k,
                                    const int64_t *k_strides, const void *a,
                                    const int64_t *a_strides, const void *b,
                                    const int64_t *b_strides, const float *a_log,
                                    const void *dt_bias, void *q_norm, void *k_norm, float *beta,
                                    float *g, int tokens, int num_heads, int head_dim,
                                    void *stream) {
  if (!q || !q_strides || !k || !k_strides || !a || !a_strides || !b || !b_strides || !a_log ||
      !dt_bias || !q_norm || !k_norm || !beta || !g)
    return WY_E_NULL;
  if (tokens < 0 || num_heads <= 0 || head_dim <= 0) return WY_E_SHAPE;
  if (head_dim != kDK) return WY_E_UNSUPPORTED;
  if (tokens == 0) return WY_OK;
  if (int64_t(tokens) * num_heads > 0x7fffffff) return WY_E_SHAPE;
  QkNormArgs p{};
  p.q = static_cast<const bf16_t *>(q);
  p.k = static_cast<const bf16_t *>(k);
  p.a = static_cast<const bf16_t *>(a);
  p.b = static_cast<const bf16_t *>(b);
  p.dt_bias = static_cast<const bf16_t *>(dt_bias);
  p.a_log = a_log;
  p.q_t = q_strides[0]; p.q_h = q_strides[1]; p.q_d = q_strides[2];
  p.k_t = k_strides[0]; p.k_h = k_strides[1]; p.k_d = k_strides[2];
  p.a_t = a_strides[0]; p.a_h = a_strides[1];
  p.b_t = b_strides[0]; p.b_h = b_strides[1];
  p.qn = static_cast<bf16_t *>(q_norm);
  p.kn = static_cast<bf16_t *>(k_norm);
  p.qn_t = p.kn_t = int64_t(num_heads) * kDK;
  p.qn_h = p.kn_h = kDK;
  p.beta = beta;
  p.g = g;
  p.heads = num_heads;
  p.q_scale = float(1.0 / sqrt(double(head_dim)));
  const int pairs = tokens * num_heads;
  const bool vec = p.q_d == 1 && p.k_d == 1 && ((p.q_t | p.q_h | p.k_t | p.k_h) & 7) == 0 &&
                   wyh::aligned16(q) && wyh::aligned16(k) && wyh::aligned16(q_norm) &&
                   wyh::aligned16(k_norm);
  if (vec && pairs >= kVecRows)
    gdn_qk_norm_gates_vec_kernel<<<unsigned((pairs + 7) / 8), 256, 0,
                                   static_cast<hipStream_t>(stream)>>>(p, pairs);
  else
    gdn_qk_norm_gates_kernel<<<unsigned(pairs), 256, 0, static_cast<hipStream_t>(stream)>>>(p);
  return wyh::launch_status();
}

extern "C" int wy_gdn_gated_rmsnorm(const void *x, const int64_t *x_strides, const void *z,
                                    const int64_t *z_strides, const float *weight, void *out,
                                    int tokens, int num_heads, int head_dim, void *stream) {
  if (!x || !x_strides || !z || !z_strides || !weight || !out) return WY_E_NULL;
  if (tokens < 0 || num_heads <= 0 || head_dim <= 0) return WY_E_SHAPE;
  if (head_dim != kDK) return WY_E_UNSUPPORTED;
  if (tokens == 0) return WY_OK;
  if (int64_t(tokens) * num_heads > 0x7fffffff) return WY_E_SHAPE;
  const int rows = tokens * num_heads;
  const bool vec = x_strides[2] == 1 && z_strides[2] == 1 &&
                   ((x_strides[0] | x_strides[1] | z_strides[0] | z_strides[1]) & 7) == 0 &&
                   wyh::aligned16(x) && wyh::aligned16(z) && wyh::aligned16(weight) &&
                   wyh::aligned16(out);
  if (vec && rows >= kVecRows)
    gdn_gated_rmsnorm_vec_kernel<<<unsigned((rows + 15) / 16), 256, 0,
                                   static_cast<hipStream_t>(stream)>>>(
        static_cast<const bf16_t *>(x), x_strides[0], x_strides[1],
        static_cast<const bf16_t *>(z), z_strides[0], z_strides[1], weight,
        static_cast<bf16_t *>(out), num_heads, rows);
  else
    gdn_gated_rmsnorm_kernel<<<unsigned(rows), 128, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const bf16_t *>(x), x_strides[0], x_strides[1], x_strides[2],
        static_cast<const bf16_t *>(z), z_strides[0], z_strides[1], z_strides[2], weight,
        static_cast<bf16_t *>(out), num_heads);
  return wyh::launch_status();
}

extern "C" int wy_gdn_decode_block(const void *fused, int64_t fused_stride0, void *conv_state,
                                   const int64_t *conv_state_strides, const void *conv_weight,
                                   int64_t conv_weight_stride0, const float *a_log,
                                   const void *dt_bias, const float *norm_weight, float *state,
                                   const int64_t *state_strides, void *out, int64_t out_stride0,
                                   int batch, int num_heads, int head_dim, void *stream) {
  if (!fused || !conv_state || !conv_state_strides || !conv_weight || !a_log || !dt_bias ||
      !norm_weight || !state || !state_strides || !out)
    return WY_E_NULL;
  if (batch < 0 || num_heads <= 0 || head_dim <= 0) return WY_E_SHAPE;
  if (head_dim != kDK) return WY_E_UNSUPPORTED;
  if (conv_state_strides[2] != 1 || state_strides[3] != 1 || state_strides[2] % 4 ||
      state_strides[1] % 4 || state_strides[0] % 4 || !wyh::aligned16(state))
    return WY_E_LAYOUT;
  if (batch == 0) return WY_OK;
  BlockArgs p{};
  p.fused = static_cast<const bf16_t *>(fused);
  p.f_b = fused_stride0;
  p.conv_state = static_cast<bf16_t *>(conv_state);
  p.cs_b = conv_state_strides[0];
  p.cs_k = conv_state_strides[1];
  p.conv_w = static_cast<const bf16_t *>(conv_weight);
  p.cw_k = conv_weight_stride0;
  p.a_log = a_log;
  p.dt_bias = static_cast<const bf16_t *>(dt_bias);
  p.norm_w = norm_weight;
  p.state = state;
  p.s_b = state_strides[0];
  p.s_h = state_strides[1];
  p.s_k = state_strides[2];
  p.out = static_cast<bf16_t *>(out);
  p.o_b = out_stride0;
  p.heads = num_heads;
  p.q_scale = float(1.0 / sqrt(double(head_dim)));
  gdn_decode_block_kernel<<<unsigned(batch * num_heads), 512, 0,
                            static_cast<hipStream_t>(stream)>>>(p);
  return wyh::launch_status();
}

extern "C" int wy_depthwise_causal_conv4_prefill(const void *x, const int64_t *x_strides,
                                                 const void *weight, int64_t w_stride_c,
                                                 int64_t w_stride_k, void *out,
                                                 const int64_t *out_strides,
                                                 const int32_t *seq_start, int tokens,
                                                 int channels, void *stream) {
  if (!x || !x_strides || !weight || !out || !out_strides) return WY_E_NULL;
  if (tokens < 0 || channels < 0) return WY_E_SHAPE;
  if (tokens == 0 || channels == 0) return WY_OK;
  const unsigned runs = unsigned((tokens + kConvRun - 1) / kConvRun);
  if (x_strides[1] == 1 && out_strides[1] == 1 && channels % 8 == 0 &&
      ((x_strides[0] | out_strides[0]) & 7) == 0 && wyh::aligned16(x) && wyh::aligned16(out)) {
    conv4_prefill_vec_kernel<<<dim3(unsigned((channels / 8 + 255) / 256), runs), 256, 0,
                               static_cast<hipStream_t>(stream)>>>(
        static_cast<const bf16_t *>(x), x_strides[0], static_cast<const bf16_t *>(weight),
        w_stride_c, w_stride_k, static_cast<bf16_t *>(out), out_strides[0], seq_start, tokens,
        channels);
    return wyh::launch_status();
  }
  const dim3 grid(unsigned((channels + 255) / 256), runs);
  conv4_prefill_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(x), x_strides[0], x_strides[1],
      static_cast<const bf16_t *>(weight), w_stride_c, w_stride_k, static_cast<bf16_t *>(out),
      out_strides[0], out_strides[1], seq_start, tokens, channels);
  return wyh::launch_status();
}

extern "C" int wy_conv_state_from_packed_prefill(void *state, const int64_t *state_strides,
                                                 const void *x, const int64_t *x_strides,
                                                 const int32_t *cu_seqlens, int batch,
                                                 int channels, void *stream) {
  if (!state || !state_strides || !x || !x_strides || !cu_seqlens) return WY_E_NULL;
  if (batch < 0 || channels < 0) return WY_E_SHAPE;
  if (state_strides[2] != 1 || x_strides[1] != 1) return WY_E_LAYOUT;
  if (batch == 0 || channels == 0) return WY_OK;
  const dim3 grid(unsigned((channels + 255) / 256), unsigned(batch));
  conv_state_pack_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(x), x_strides[0], static_cast<bf16_t *>(state),
      state_strides[0], state_strides[1], cu_seqlens, channels);
  return wyh::launch_status();
}
