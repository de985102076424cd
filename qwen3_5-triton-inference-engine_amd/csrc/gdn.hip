// Gated DeltaNet (GDN) delta-rule recurrence on gfx950: the decode update of
// the cached state and the varlen sequential prefill.
//
// Per token t and value head h, with the state S [DK, DV] fp32:
//   S      = exp(g_t) * S
//   mem    = k_t^T S                         [DV]
//   delta  = beta_t * (v_t - mem)            [DV]
//   S      = S + k_t delta^T
//   out_t  = q_t^T S                         [DV]  (stored as bf16)
// Reference: gdn_recurrent_prefill.py:52-143 (sequential kernel), :151-246
// (decode kernel), ops :1050-1146 and :1185-1260.
//
// The lane layout and the step itself are in gdn_common.h.  The output uses q^T S_new = q^T S_decayed + (q^T k) delta, the same value
// as the reference's q^T S_new, so the two reductions of a token (k^T S and
// q^T S, plus q^T k) run together, before the update.
#include "gdn_common.h"

using namespace wy;
using namespace wy::gdn;

namespace {

// Tokens whose inputs are in flight in the prefill: deep for the latency-
// bound narrow layout, shallow for the wide one (registers set occupancy),
// and the wave count (16-column waves) below which the narrow layout is
// used.  Build-time tunables (-D) for measurement; the defaults are the
// measured best.
#ifndef WY_GDN_PREFETCH_NARROW
#define WY_GDN_PREFETCH_NARROW 4
#endif
#ifndef WY_GDN_PREFETCH_WIDE
#define WY_GDN_PREFETCH_WIDE 2
#endif
#ifndef WY_GDN_NARROW_BELOW
#define WY_GDN_NARROW_BELOW 2048
#endif
template <int NC>
constexpr int prefetch_depth() { return NC == 1 ? WY_GDN_PREFETCH_NARROW : WY_GDN_PREFETCH_WIDE; }

__device__ __forceinline__ float *state_block(const GdnArgs &a, int b, int h, int kg, int col) {
  return a.state + b * a.s_b + h * a.s_h + int64_t(kg * kRows) * a.s_k + col;
}

// Decode: one token per sequence, S read from and written back to the cache.
// Workgroup = 8 wavefronts = 128 value columns of one (sequence, head); all
// 8 state loads of a lane are issued before the first use.
template <bool kContig>
__global__ __launch_bounds__(512) void gdn_recurrent_decode_kernel(const GdnArgs a) {
  const int bh = blockIdx.x;
  const int b = bh / a.heads, h = bh - b * a.heads;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kg = lane & 15, cg = lane >> 4;
  const int col = blockIdx.y * 128 + wave * kWaveCols + cg * kCols;
  float *sp = state_block(a, b, h, kg, col);
  float s[kRows][kCols];
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const float4 x = *reinterpret_cast<const float4 *>(sp + i * a.s_k);
    s[i][0] = x.x;
    s[i][1] = x.y;
    s[i][2] = x.z;
    s[i][3] = x.w;
  }
  TokenIn in;
  load_token<kContig>(a, b, h, kg, col, in);
  float o[kCols];
  gdn_step(s, in, o);
#pragma unroll
  for (int i = 0; i < kRows; ++i)
    *reinterpret_cast<float4 *>(sp + i * a.s_k) = make_float4(s[i][0], s[i][1], s[i][2], s[i][3]);
  if (kg == 0) store4<kContig>(a.out + b * a.o_t + h * a.o_h + col * a.o_d, a.o_d, o);
}

// Varlen sequential prefill: one wavefront per (sequence, head, 16 value
// columns), walking its sequence's tokens in order from a zero state; the
// inputs of the next kPrefetch tokens are in flight during each update.  The
// state is kept lazily decayed (gdn_step_scaled).
template <bool kContig, int NC>
__global__ __launch_bounds__(64) void gdn_prefill_sequential_kernel(const GdnArgs a, int batch) {
  // grid: sequence fastest, then head, then column block
  const int b = blockIdx.x % batch;
  const int h = (blockIdx.x / batch) % a.heads;
  const int vb = blockIdx.x / (batch * a.heads);
  const int lane = threadIdx.x;
  const int kg = lane & 15, cg = lane >> 4;
  const int col = vb * 4 * NC + cg * NC;
  const int start = a.cu_seqlens[b];
  const int len = a.cu_seqlens[b + 1] - start;
  float s[kRows][NC];
  float c = 1.f;  // the state is c * s (gdn_step_scaled)
#pragma unroll
  for (int i = 0; i < kRows; ++i)
#pragma unroll
    for (int j = 0; j < NC; ++j) s[i][j] = 0.f;
  // kPrefetch tokens in flight: token t's inputs are requested while token
  // t - kPrefetch is processed, so the load latency hides behind several steps.
  // Every load and store of the main loop is unconditional (a prefetch past
  // the end re-reads the last token; all 16 lanes of a row store the same
  // output values), so the compiler's memory counter waits name exactly the
  // token a step needs: a load or store that only some paths issue makes it
  // wait for everything in flight.
  constexpr int kPrefetch = prefetch_depth<NC>();
  auto store_out = [&](int t, const float (&o)[NC]) {
    bf16_t *op = a.out + (start + t) * a.o_t + h * a.o_h + col * a.o_d;
    if constexpr (NC == kCols)
      store4<kContig>(op, a.o_d, o);
    else
#pragma unroll
      for (int e = 0; e < NC; ++e) op[e * a.o_d] = bf16_t(f32_to_bf16_bits(o[e]));
  };
  if (len > 0) {
    TokenRaw<NC> buf[kPrefetch];
#pragma unroll
    for (int u = 0; u < kPrefetch; ++u)
      load_token_raw<kContig, NC>(a, start + min(u, len - 1), h, kg, col, buf[u]);
    const int nfull = len - len % kPrefetch;
    for (int t0 = 0; t0 < nfull; t0 += kPrefetch) {
#pragma unroll
      for (int u = 0; u < kPrefetch; ++u) {
        float o[NC];
        gdn_step_scaled(s, c, unpack_token(buf[u]), o);
        store_out(t0 + u, o);
        load_token_raw<kContig, NC>(a, start + min(t0 + u + kPrefetch, len - 1), h, kg, col,
                                    buf[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kPrefetch - 1; ++u)
      if (nfull + u < len) {
        float o[NC];
        gdn_step_scaled(s, c, unpack_token(buf[u]), o);
        store_out(nfull + u, o);
      }
  }
  float *sp = state_block(a, b, h, kg, col);
#pragma unroll
  for (int i = 0; i < kRows; ++i)
#pragma unroll
    for (int j = 0; j < NC; ++j) sp[i * a.s_k + j] = c * s[i][j];
}

// Shared argument checks; returns WY_OK and fills a, or an error code.
int gdn_setup(GdnArgs &a, bool &contig, const void *q, const int64_t *qs, const void *k,
              const int64_t *ks, const void *v, const int64_t *vs, const float *beta,
              const int64_t *bs, const float *g, const int64_t *gs, void *out,
              const int64_t *os, float *state, const int64_t *ss, int heads, int key_dim,
              int value_dim) {
  if (!q || !qs || !k || !ks || !v || !vs || !beta || !bs || !g || !gs || !out || !os ||
      !state || !ss)
    return WY_E_NULL;
  if (heads <= 0 || key_dim <= 0 || value_dim <= 0) return WY_E_SHAPE;
  if (key_dim != kDK || value_dim % 128 != 0) return WY_E_UNSUPPORTED;
  if (ss[3] != 1 || ss[2] % 4 || ss[1] % 4 || ss[0] % 4 || !wyh::aligned16(state))
    return WY_E_LAYOUT;
  a = GdnArgs{};
  a.q = static_cast<const bf16_t *>(q);
  a.k = static_cast<const bf16_t *>(k);
  a.v = static_cast<const bf16_t *>(v);
  a.q_t = qs[0]; a.q_h = qs[1]; a.q_d = qs[2];
  a.k_t = ks[0]; a.k_h = ks[1]; a.k_d = ks[2];
  a.v_t = vs[0]; a.v_h = vs[1]; a.v_d = vs[2];
  a.beta = beta; a.beta_t = bs[0]; a.beta_h = bs[1];
  a.g = g; a.g_t = gs[0]; a.g_h = gs[1];
  a.out = static_cast<bf16_t *>(out);
  a.o_t = os[0]; a.o_h = os[1]; a.o_d = os[2];
  a.state = state;
  a.s_b = ss[0]; a.s_h = ss[1]; a.s_k = ss[2]; a.s_v = ss[3];
  a.heads = heads;
  a.dv = value_dim;
  // 16-byte q/k rows (8 bf16 per lane) and 8-byte v / out quads
  contig = qs[2] == 1 && ks[2] == 1 && vs[2] == 1 && os[2] == 1 && qs[0] % 8 == 0 &&
           qs[1] % 8 == 0 && ks[0] % 8 == 0 && ks[1] % 8 == 0 && wyh::aligned16(q) &&
           wyh::aligned16(k) && vs[0] % 4 == 0 && vs[1] % 4 == 0 && os[0] % 4 == 0 &&
           os[1] % 4 == 0 && (reinterpret_cast<uintptr_t>(v) & 7u) == 0 &&
           (reinterpret_cast<uintptr_t>(out) & 7u) == 0;
  return WY_OK;
}

}  // namespace

extern "C" int wy_gdn_recurrent_decode(const void *q, const int64_t *q_strides, const void *k,
                                       const int64_t *k_strides, const void *v,
                                       const int64_t *v_strides, const float *beta,
                                       const int64_t *beta_strides, const float *g,
                                       const int64_t *g_strides, void *out,
                                       const int64_t *out_strides, float *state,
                                       const int64_t *state_strides, int batch, int num_heads,
                                       int key_dim, int value_dim, void *stream) {
  GdnArgs a;
  bool contig = false;
  const int rc = gdn_setup(a, contig, q, q_strides, k, k_strides, v, v_strides, beta,
                           beta_strides, g, g_strides, out, out_strides, state, state_strides,
                           num_heads, key_dim, value_dim);
  if (rc != WY_OK) return rc;
  if (batch < 0) return WY_E_SHAPE;
  if (batch == 0) return WY_OK;
  const dim3 grid(unsigned(batch * num_heads), unsigned(value_dim / 128));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (contig)
    gdn_recurrent_decode_kernel<true><<<grid, 512, 0, st>>>(a);
  else
    gdn_recurrent_decode_kernel<false><<<grid, 512, 0, st>>>(a);
  return wyh::launch_status();
}

extern "C" int wy_gdn_recurrent_prefill_sequential(
    const void *q, const int64_t *q_strides, const void *k, const int64_t *k_strides,
    const void *v, const int64_t *v_strides, const float *beta, const int64_t *beta_strides,
    const float *g, const int64_t *g_strides, void *out, const int64_t *out_strides,
    float *state, const int64_t *state_strides, const int32_t *cu_seqlens, int batch,
    int num_heads, int key_dim, int value_dim, void *stream) {
  GdnArgs a;
  bool contig = false;
  const int rc = gdn_setup(a, contig, q, q_strides, k, k_strides, v, v_strides, beta,
                           beta_strides, g, g_strides, out, out_strides, state, state_strides,
                           num_heads, key_dim, value_dim);
  if (rc != WY_OK) return rc;
  if (!cu_seqlens) return WY_E_NULL;
  if (batch < 0) return WY_E_SHAPE;
  if (batch == 0) return WY_OK;
  a.cu_seqlens = cu_seqlens;
  // 16 value columns per wavefront (4 per lane) when the grid fills the
  // chip several times over; else 4 per wavefront (1 per lane): a token step
  // is a chain of dependent VALU / DPP work, so fewer columns per lane
  // shorten the chain where there are SIMDs to spare.
  const int64_t wide = int64_t(batch) * num_heads * (value_dim / kWaveCols);
  const bool narrow = wide < WY_GDN_NARROW_BELOW;
  const int64_t blocks = narrow ? wide * 4 : wide;
  if (blocks > 0x7fffffff) return WY_E_SHAPE;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (narrow) {
    if (contig)
      gdn_prefill_sequential_kernel<true, 1><<<unsigned(blocks), 64, 0, st>>>(a, batch);
    else
      gdn_prefill_sequential_kernel<false, 1><<<unsigned(blocks), 64, 0, st>>>(a, batch);
  } else {
    if (contig)
      gdn_prefill_sequential_kernel<true, kCols><<<unsigned(blocks), 64, 0, st>>>(a, batch);
    else
      gdn_prefill_sequential_kernel<false, kCols><<<unsigned(blocks), 64, 0, st>>>(a, batch);
  }
  return wyh::launch_status();
}
