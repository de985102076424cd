// Gated DeltaNet chunk-64 (WY) prefill on gfx950: the delta-rule recurrence of
// one long prompt in three launches instead of a token-by-token walk.
// Reference: gdn_recurrent_prefill.py:249-402 (prepare kernel), :405-562 (state),
// :565-690 (output); ops :707-1023, the chain :1026-1051.
//
// Per chunk of 64 tokens and head, with G = cumsum(g) inside the chunk:
//   L[t, i] = beta_t exp(G_t - G_i) <k_t, k_i>   (i < t)
//   u_base  = (I + L)^-1 (beta v),   w = (I + L)^-1 (beta exp(G) k)
//   delta   = u_base - w S_c                       (S_c: state entering chunk c)
//   S_c+1   = exp(G_last) S_c + k^T (delta exp(G_last - G_t))
//   out_t   = exp(G_t) q_t S_c + sum_{i <= t} exp(G_t - G_i) <q_t, k_i> delta_i
// Tokens past T count as beta = g = 0, k = v = q = 0 (their rows are zero).
//
// Precision: <k_t, k_i> and <q_t, k_i> are bf16 x bf16 products summed in
// fp32 on v_mfma_f32_32x32x16_bf16 (exact products).  In the chunk recurrence
// every fp32 operand x is split as hi = bf16(x), lo = bf16(x - hi) (16 bits
// of mantissa) and a product of two fp32 operands is hi*hi + hi*lo + lo*hi on
// v_mfma_f32_16x16x32_bf16 (relative error ~2^-16; the reference uses
// three-pass tf32 for the same products); a bf16 x fp32 product is two such
// MFMAs; the output kernel's fp32 operands are split the same way.
// (I + L)^-1 is applied by forward substitution on the right-hand sides, one
// column per thread, in fp32.
#include "wy_common.h"

using namespace wy;

namespace {

constexpr int kC = 64;    // chunk tokens
constexpr int kDK = 128;  // key dim
constexpr int kDV = 128;  // value dim
constexpr int kBV = 16;   // value columns per state workgroup
constexpr int kKPad = kDK + 8;

typedef float f32x4_t_ __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t_ mfma16x32(u32x4_t a, u32x4_t b, f32x4_t_ c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
// fp32 x = hi + lo + O(2^-17 |x|) with hi = bf16(x), lo = bf16(x - hi): eight
// values split into two bf16 MFMA operands
__device__ __forceinline__ void split8(const float (&x)[8], u32x4_t &hi, u32x4_t &lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float h0 = round_bf16(x[2 * e]), h1 = round_bf16(x[2 * e + 1]);
    hi[e] = pack_bf16x2(h0, h1);
    lo[e] = pack_bf16x2(x[2 * e] - h0, x[2 * e + 1] - h1);
  }
}

// kk^T-type 64 x 64 product of two bf16 [64][kKPad] LDS tiles on 32x32x16
// MFMAs: wave w computes output tile (w / 2, w % 2); register r of lane l is
// row 32 (w/2) + (r&3) + 8 (r>>2) + 4 (l/32), column 32 (w%2) + l%32.
__device__ __forceinline__ f32x16_t gram64(const bf16_t (*a)[kKPad], const bf16_t (*b)[kKPad],
                                           int wave, int lane) {
  const int r0 = 32 * (wave >> 1), c0 = 32 * (wave & 1);
  f32x16_t acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
  for (int ks = 0; ks < kDK / 16; ++ks) {
    const u32x4_t av = ld16(&a[r0 + (lane & 31)][ks * 16 + 8 * (lane >> 5)]);
    const u32x4_t bv = ld16(&b[c0 + (lane & 31)][ks * 16 + 8 * (lane >> 5)]);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, av),
                                                  __builtin_bit_cast(bf16x8_t, bv), acc, 0, 0, 0);
  }
  return acc;
}

// Rows [t0, t0 + nval) of a [T, H, 128] bf16 tensor (head h) into LDS; rows
// past nval are zero.  Inner stride 1, rows 16-byte aligned (host-checked).
__device__ __forceinline__ void load_rows(bf16_t (*dst)[kKPad], const bf16_t *src, int64_t st,
                                          int nval) {
  for (int i = threadIdx.x; i < kC * 16; i += 256) {
    const int r = i >> 4, c = (i & 15) * 8;
    u32x4_t x = {0u, 0u, 0u, 0u};
    if (r < nval) x = ld16(src + r * st + c);
    st16(&dst[r][c], x);
  }
}

// ---- 1. prepare: G, w, u_base per (chunk, head) ----------------------------------
__global__ __launch_bounds__(256) void gdn_chunk_prepare_kernel(
    const bf16_t *__restrict__ k, int64_t k_t, int64_t k_h, const bf16_t *__restrict__ v,
    int64_t v_t, int64_t v_h, const float *__restrict__ beta, int64_t b_t, int64_t b_h,
    const float *__restrict__ g, int64_t g_t, int64_t g_h, float *__restrict__ w,
    float *__restrict__ u, float *__restrict__ gcs, int T, int H) {
  __shared__ __align__(16) bf16_t ks[kC][kKPad];
  __shared__ __align__(16) bf16_t vs[kC][kKPad];
  __shared__ __align__(16) float L[kC][kC + 4];
  __shared__ float sb[kC], sG[kC], seG[kC];
  const int n = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int t0 = n * kC;
  const int nval = min(kC, T - t0);
  load_rows(ks, k + int64_t(t0) * k_t + h * k_h, k_t, nval);
  load_rows(vs, v + int64_t(t0) * v_t + h * v_h, v_t, nval);
  if (tid < kC) {
    const bool ok = tid < nval;
    const float bt = ok ? beta[int64_t(t0 + tid) * b_t + h * b_h] : 0.f;
    float G = ok ? g[int64_t(t0 + tid) * g_t + h * g_h] : 0.f;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {  // inclusive prefix sum over the chunk
      const float y = __shfl_up(G, o);
      if (tid >= o) G += y;
    }
    sb[tid] = bt;
    sG[tid] = G;
    seG[tid] = expf(G);
    gcs[(int64_t(n) * H + h) * kC + tid] = G;
  }
  __syncthreads();

  // L = beta_t exp(G_t - G_i) <k_t, k_i>, strictly lower, in LDS
  if (wave != 1) {  // output tile (0, 1) lies above the diagonal
    const f32x16_t kk = gram64(ks, ks, wave, lane);
    const int i = 32 * (wave & 1) + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 32 * (wave >> 1) + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
      L[t][i] = (i < t && t < nval) ? sb[t] * expf(sG[t] - sG[i]) * kk[r] : 0.f;
    }
  } else {
    for (int e = lane; e < 32 * 32; e += 64) L[e >> 5][32 + (e & 31)] = 0.f;
  }
  __syncthreads();

  // forward substitution X = (I + L)^-1 B, thread c owning column c of
  // B = [beta v | beta exp(G) k]: X_t = B_t - sum_{i<t} L[t][i] X_i
  const int c = tid;
  float x[kC];
#pragma unroll
  for (int t = 0; t < kC; ++t) {
    float acc = c < kDV ? sb[t] * bf16_to_f32(vs[t][c]) : sb[t] * seG[t] * bf16_to_f32(ks[t][c - kDV]);
#pragma unroll
    for (int i4 = 0; i4 < t; i4 += 4) {
      const float4 l4 = *reinterpret_cast<const float4 *>(&L[t][i4]);
      acc -= l4.x * x[i4];
      if (i4 + 1 < t) acc -= l4.y * x[i4 + 1];
      if (i4 + 2 < t) acc -= l4.z * x[i4 + 2];
      if (i4 + 3 < t) acc -= l4.w * x[i4 + 3];
    }
    x[t] = acc;
  }
  float *dst = (c < kDV ? u : w) + (int64_t(n) * H + h) * kC * 128 + (c & 127);
#pragma unroll
  for (int t = 0; t < kC; ++t) dst[t * 128] = x[t];
}

// ---- 2. state: the chunk recurrence per (head, 16 value columns) ----------------
//
// S (128 x 16 fp32) lives in registers in the 16x16 MFMA output layout: wave
// wv holds key rows 32 wv .. 32 wv + 31 as two 16-row tiles; lane l has rows
// 16 dt + 4 (l/16) + j, column l%16.  Per chunk:
//   delta (64 x 16) = u_base - w S     wave wv: token rows 16 wv .. +15
//   dd = delta * exp(G_last - G_t)     (zero past T)
//   S = exp(G_last) S + k^T dd
// The shared B operands (S of w S, dd of k^T dd) are split into bf16 hi/lo
// once, by the lanes that own them, and published to LDS transposed
// ([column][k index]) so that each lane's 8 consecutive k indices are one
// 16-byte read.  The k index of an MFMA may be any permutation shared by its
// A and B operands: in w S lane (row r, group qd) takes keys 32 qd .. 32 qd +
// 31, so its w operand is 32 consecutive floats of row r (one contiguous
// load, fetched a chunk ahead); in k^T dd it takes tokens 16 qd .. 16 qd + 15
// and reads its k operand (8 tokens of one key row) from the row-major k
// tile with two transposing reads.
constexpr int kSPad = kDK + 8;   // bf16 row pitch of the transposed S
constexpr int kDPad = kC + 8;    // bf16 row pitch of the transposed dd

__device__ __forceinline__ u32x2_t lds_read_tr16(const bf16_t *p) {
  typedef short i16x4_t __attribute__((ext_vector_type(4)));
  const i16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4_t *)(p));
  return __builtin_bit_cast(u32x2_t, r);
}

// four fp32 values -> (hi, lo) bf16 quads, x = hi + lo + O(2^-17 |x|)
__device__ __forceinline__ void split4(const f32x4_t_ x, u32x2_t &hi, u32x2_t &lo) {
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint32_t hp = pack_bf16x2(x[2 * e], x[2 * e + 1]);
    hi[e] = hp;
    lo[e] = pack_bf16x2(x[2 * e] - __uint_as_float(hp << 16),
                        x[2 * e + 1] - __uint_as_float(hp & 0xffff0000u));
  }
}

// Two wave roles.  Waves 0-3 compute, as above, from LDS only.  Waves 4-7
// move the data: they issue the global loads of chunk c + 2 at the start of
// chunk c (two register sets), store chunk c's entering state and delta rows from LDS, and write
// the loaded chunk into the other half of a double buffer before the chunk's
// last barrier, with the decay factors exp(G_last - G_t) (zero past T) and
// exp(G_last) computed once.  A CU streams only ~50 GB/s from L2, so the 56 KB a chunk
// moves per workgroup takes about as long as the chunk's arithmetic; with
// the roles split the two overlap instead of adding up.
constexpr int kWPad = kDK + 4;   // fp32 row pitch of the w tile
constexpr int kFPad = kDK + 4;   // fp32 row pitch of the transposed S (state store)
struct StateLds {
  float w[2][kC][kWPad];         // w of the chunk (A operand rows)
  bf16_t k[2][kC][kKPad];        // k of the chunk, row-major
  float u[2][kC][kBV];           // u_base columns v0 .. v0 + 15
  float E[2][kC];                // exp(G_last - G_t), zero past T
  float eg[4];                   // exp(G_last) (4: keeps the members after it 16-byte aligned)
  bf16_t Sh[kBV][kSPad], Sl[kBV][kSPad];   // S^T hi / lo: B operand of w S
  bf16_t Dh[kBV][kDPad], Dl[kBV][kDPad];   // dd^T hi / lo: B operand of k^T dd
  float dl[kC][kBV];             // delta rows for the store
  float Sf[kBV][kFPad];          // S^T fp32 for the state store
};
constexpr int kStateLds = int(sizeof(StateLds));
static_assert(offsetof(StateLds, Sh) % 16 == 0 && offsetof(StateLds, Dh) % 16 == 0 &&
                  offsetof(StateLds, dl) % 16 == 0 && offsetof(StateLds, Sf) % 16 == 0,
              "16-byte LDS accesses");
static_assert(kStateLds <= 160 * 1024, "state kernel LDS");

__global__ __launch_bounds__(512) void gdn_chunk_state_kernel(
    const bf16_t *__restrict__ k, int64_t k_t, int64_t k_h, const float *__restrict__ w,
    const float *__restrict__ u, const float *__restrict__ gcs, float *__restrict__ delta,
    float *__restrict__ chunk_state, float *__restrict__ final_state, int T, int H, int N) {
  extern __shared__ __align__(16) unsigned char state_smem[];
  StateLds &L = *reinterpret_cast<StateLds *>(state_smem);
  const int h = blockIdx.x, v0 = blockIdx.y * kBV, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const bool mover = wave >= 4;
  const int ptid = tid - 256;   // mover thread index

  // mover: chunk c's global loads into register set sl / into LDS buffer b
  f32x4_t_ rw[2][8];
  u32x4_t rk[2][4];
  f32x4_t_ ru[2];
  float rG[2] = {0.f, 0.f};
  auto load = [&](int c, int sl) {
    const float *wc = w + (int64_t(c) * H + h) * kC * kDK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = ptid + 256 * i;
      rw[sl][i] = *reinterpret_cast<const f32x4_t_ *>(wc + (e >> 5) * kDK + (e & 31) * 4);
    }
    const int t0 = c * kC, last = min(kC, T - t0) - 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = ptid + 256 * i, r = min(e >> 4, last);   // rows past T: zeroed at the write
      rk[sl][i] = ld16(k + int64_t(t0 + r) * k_t + h * k_h + (e & 15) * 8);
    }
    ru[sl] = *reinterpret_cast<const f32x4_t_ *>(u + ((int64_t(c) * H + h) * kC + (ptid >> 2)) * kDV +
                                             v0 + (ptid & 3) * 4);
    if (ptid < kC) rG[sl] = gcs[(int64_t(c) * H + h) * kC + ptid];
  };
  auto put = [&](int c, int b, int sl) {
    const int nval = min(kC, T - c * kC);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = ptid + 256 * i;
      *reinterpret_cast<f32x4_t_ *>(&L.w[b][e >> 5][(e & 31) * 4]) = rw[sl][i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = ptid + 256 * i;
      st16(&L.k[b][e >> 4][(e & 15) * 8], (e >> 4) < nval ? rk[sl][i] : u32x4_t{0u, 0u, 0u, 0u});
    }
    *reinterpret_cast<f32x4_t_ *>(&L.u[b][ptid >> 2][(ptid & 3) * 4]) = ru[sl];
    const float G_last = __shfl(rG[sl], kC - 1);   // mover threads 0..63 are one wave
    if (ptid < kC) L.E[b][ptid] = ptid < nval ? expf(G_last - rG[sl]) : 0.f;
    if (ptid == 0) L.eg[b] = expf(G_last);
  };

  // compute waves: S rows 32 wave + 4 quad + j (S0) and + 16 (S1), column col
  const int col = lane & 15, quad = lane >> 4;
  const int dS = 32 * wave + 4 * quad;
  f32x4_t_ S0 = {0.f, 0.f, 0.f, 0.f}, S1 = {0.f, 0.f, 0.f, 0.f};

  if (mover) {
    load(0, 0);
    put(0, 0, 0);
    if (N > 1) load(1, 1);
  }
  __syncthreads();
  for (int c0 = 0; c0 < N; c0 += 2)
#pragma unroll
  for (int b = 0; b < 2; ++b) {   // chunk c uses LDS buffer and register set c & 1
    const int c = c0 + b;
    if (c >= N) break;   // uniform over the workgroup
    // ---- phase 1: publish S; the mover requests chunk c + 2
    if (mover) {
      if (c + 2 < N) load(c + 2, b);
    } else {
      u32x2_t h0, l0, h1, l1;
      split4(S0, h0, l0);
      split4(S1, h1, l1);
      *reinterpret_cast<u32x2_t *>(&L.Sh[col][dS]) = h0;
      *reinterpret_cast<u32x2_t *>(&L.Sl[col][dS]) = l0;
      *reinterpret_cast<u32x2_t *>(&L.Sh[col][dS + 16]) = h1;
      *reinterpret_cast<u32x2_t *>(&L.Sl[col][dS + 16]) = l1;
      *reinterpret_cast<f32x4_t_ *>(&L.Sf[col][dS]) = S0;
      *reinterpret_cast<f32x4_t_ *>(&L.Sf[col][dS + 16]) = S1;
    }
    __syncthreads();
    // ---- phase 2: delta = u_base - w S and dd; the mover stores the entering state
    if (mover) {
      float *cs = chunk_state + (int64_t(c) * H + h) * kDK * kDV + v0;
      const int cc = ptid & 15;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int d = 4 * ((ptid >> 4) + 16 * i);
        const f32x4_t_ x = *reinterpret_cast<const f32x4_t_ *>(&L.Sf[cc][d]);
#pragma unroll
        for (int e = 0; e < 4; ++e) cs[(d + e) * kDV + cc] = x[e];
      }
    } else {
      // w S on bf16 MFMAs with both fp32 operands split (hi hi + hi lo + lo hi);
      // step ks covers keys 32 qd + 8 ks .. +7 of lane group qd
      f32x4_t_ acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const float *wr = &L.w[b][16 * wave + col][32 * quad + 8 * ks];
        const f32x4_t_ x0 = *reinterpret_cast<const f32x4_t_ *>(wr);
        const f32x4_t_ x1 = *reinterpret_cast<const f32x4_t_ *>(wr + 4);
        const u32x4_t bh = ld16(&L.Sh[col][32 * quad + 8 * ks]);
        const u32x4_t bl = ld16(&L.Sl[col][32 * quad + 8 * ks]);
        u32x2_t ah0, al0, ah1, al1;
        split4(x0, ah0, al0);
        split4(x1, ah1, al1);
        const u32x4_t ah = {ah0[0], ah0[1], ah1[0], ah1[1]};
        const u32x4_t al = {al0[0], al0[1], al1[0], al1[1]};
        acc = mfma16x32(ah, bh, acc);
        acc = mfma16x32(ah, bl, acc);
        acc = mfma16x32(al, bh, acc);
      }
      const f32x4_t_ ex = *reinterpret_cast<const f32x4_t_ *>(&L.E[b][16 * wave + 4 * quad]);
      f32x4_t_ dd;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * wave + 4 * quad + j;
        const float d = L.u[b][t][col] - acc[j];
        L.dl[t][col] = d;
        dd[j] = d * ex[j];
      }
      u32x2_t dh, dl;
      split4(dd, dh, dl);
      *reinterpret_cast<u32x2_t *>(&L.Dh[col][16 * wave + 4 * quad]) = dh;
      *reinterpret_cast<u32x2_t *>(&L.Dl[col][16 * wave + 4 * quad]) = dl;
    }
    __syncthreads();
    // ---- phase 3: S = exp(G_last) S + k^T dd; the mover stores delta and
    // fills the other buffer with chunk c + 1
    if (mover) {
      float *dlt = delta + (int64_t(c) * H + h) * kC * kDV + v0;
      const int t = ptid >> 2, p4 = (ptid & 3) * 4;
      *reinterpret_cast<f32x4_t_ *>(dlt + t * kDV + p4) =
          *reinterpret_cast<const f32x4_t_ *>(&L.dl[t][p4]);
      if (c + 1 < N) put(c + 1, b ^ 1, b ^ 1);
    } else {
      // A[d][t] = k[t][d] (bf16, exact), dd split; step ks covers tokens
      // 16 qd + 8 ks .. +7 of lane group qd.  Transposing read: lane i of a
      // 16-lane group receives element i%4 of the 4-token pieces addressed by
      // lanes 4j + i/4, so lane L addresses token row t0 + L/4 at key 4 (L%4)
      // of the tile's 16 keys.
      const float eg = L.eg[b];
      S0 *= eg;
      S1 *= eg;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int tr = 16 * quad + 8 * ks + (col >> 2), dk = 32 * wave + 4 * (col & 3);
        const u32x2_t p0 = lds_read_tr16(&L.k[b][tr][dk]), q0 = lds_read_tr16(&L.k[b][tr + 4][dk]);
        const u32x2_t p1 = lds_read_tr16(&L.k[b][tr][dk + 16]);
        const u32x2_t q1 = lds_read_tr16(&L.k[b][tr + 4][dk + 16]);
        const u32x4_t a0 = {p0[0], p0[1], q0[0], q0[1]}, a1 = {p1[0], p1[1], q1[0], q1[1]};
        const u32x4_t bh = ld16(&L.Dh[col][16 * quad + 8 * ks]);
        const u32x4_t bl = ld16(&L.Dl[col][16 * quad + 8 * ks]);
        S0 = mfma16x32(a0, bh, S0);
        S0 = mfma16x32(a0, bl, S0);
        S1 = mfma16x32(a1, bh, S1);
        S1 = mfma16x32(a1, bl, S1);
      }
    }
    __syncthreads();  // the next chunk rewrites Sh/Sl/Sf/Dh/Dl/dl and reads buffer b ^ 1
  }
  if (!mover) {
    float *fs = final_state + int64_t(h) * kDK * kDV + v0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      fs[(dS + j) * kDV + col] = S0[j];
      fs[(dS + 16 + j) * kDV + col] = S1[j];
    }
  }
}

// ---- 3. output per (chunk, head) -------------------------------------------------
//
// out (64 x 128) = exp(G_t) q S_c + A delta with A[t][i] = <q_t, k_i>
// exp(G_t - G_i) (i <= t).  Wave wv owns token rows 16 wv .. +15 and all 128
// value columns (8 tiles of 16 x 16) on v_mfma_f32_16x16x32_bf16: q is bf16
// (exact), S_c and delta are split once into bf16 hi / lo planes in LDS
// (row-major; their k index runs down the rows, so each lane's 8 consecutive
// k values come from two transposing reads), A is split in registers; q S_c
// takes 2 products per step (q S_hi + q S_lo), A delta 3 (hi hi + hi lo + lo hi).
constexpr int kOPad = kDV + 8;   // bf16 row pitch of the S_c / delta planes
struct OutLds {
  bf16_t qs[kC][kKPad];
  bf16_t ks[kC][kKPad];
  float A[kC][kC + 4];
  bf16_t Sh[kDK][kOPad], Sl[kDK][kOPad];   // S_c split (rows = keys)
  bf16_t Dh[kC][kOPad], Dl[kC][kOPad];     // delta split (rows = chunk tokens)
  float sG[kC];
};
constexpr int kOutLds = int(sizeof(OutLds));
static_assert(kOutLds <= 160 * 1024, "output kernel LDS");
static_assert(offsetof(OutLds, Sh) % 16 == 0 && offsetof(OutLds, Dh) % 16 == 0 &&
                  offsetof(OutLds, A) % 16 == 0 && offsetof(OutLds, ks) % 16 == 0,
              "16-byte LDS accesses");

__global__ __launch_bounds__(256) void gdn_chunk_output_kernel(
    const bf16_t *__restrict__ q, int64_t q_t, int64_t q_h, const bf16_t *__restrict__ k,
    int64_t k_t, int64_t k_h, const float *__restrict__ delta, const float *__restrict__ gcs,
    const float *__restrict__ chunk_state, bf16_t *__restrict__ out, int64_t o_t, int64_t o_h,
    int T, int H) {
  extern __shared__ __align__(16) unsigned char out_smem[];
  OutLds &L = *reinterpret_cast<OutLds *>(out_smem);
  const int n = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, quad = lane >> 4;
  const int t0 = n * kC;
  const int nval = min(kC, T - t0);
  // S_c and delta: 16-byte loads, split into the hi / lo planes
  const float *Sc = chunk_state + (int64_t(n) * H + h) * kDK * kDV;
  const float *dl = delta + (int64_t(n) * H + h) * kC * kDV;
  f32x4_t_ sv[16], dv[8];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int e = tid + 256 * i;
    sv[i] = *reinterpret_cast<const f32x4_t_ *>(Sc + (e >> 5) * kDV + (e & 31) * 4);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int e = tid + 256 * i;
    dv[i] = *reinterpret_cast<const f32x4_t_ *>(dl + (e >> 5) * kDV + (e & 31) * 4);
  }
  load_rows(L.qs, q + int64_t(t0) * q_t + h * q_h, q_t, nval);
  load_rows(L.ks, k + int64_t(t0) * k_t + h * k_h, k_t, nval);
  if (tid < kC) L.sG[tid] = gcs[(int64_t(n) * H + h) * kC + tid];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int e = tid + 256 * i;
    u32x2_t hi, lo;
    split4(sv[i], hi, lo);
    *reinterpret_cast<u32x2_t *>(&L.Sh[e >> 5][(e & 31) * 4]) = hi;
    *reinterpret_cast<u32x2_t *>(&L.Sl[e >> 5][(e & 31) * 4]) = lo;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int e = tid + 256 * i;
    u32x2_t hi, lo;
    split4(dv[i], hi, lo);
    *reinterpret_cast<u32x2_t *>(&L.Dh[e >> 5][(e & 31) * 4]) = hi;
    *reinterpret_cast<u32x2_t *>(&L.Dl[e >> 5][(e & 31) * 4]) = lo;
  }
  __syncthreads();
  if (wave != 1) {
    const f32x16_t qk = gram64(L.qs, L.ks, wave, lane);
    const int i = 32 * (wave & 1) + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 32 * (wave >> 1) + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
      L.A[t][i] = (i <= t && t < nval) ? qk[r] * expf(L.sG[t] - L.sG[i]) : 0.f;
    }
  } else {
    for (int e = lane; e < 32 * 32; e += 64) L.A[e >> 5][32 + (e & 31)] = 0.f;
  }
  __syncthreads();

  // B operand of k-step rows r0 .. r0 + 31 (lane group quad: rows r0 + 8 quad
  // .. +7) and value columns 16 vt .. +15 of a plane: lane L of the 16-lane
  // group addresses row r0 + 8 quad + L/4 (+4) at column 16 vt + 4 (L%4)
  const int trow = 8 * quad + (col >> 2), tcol = 4 * (col & 3);
  auto bop = [&](const bf16_t (*P)[kOPad], int r0, int vt) {
    const u32x2_t p = lds_read_tr16(&P[r0 + trow][16 * vt + tcol]);
    const u32x2_t q2 = lds_read_tr16(&P[r0 + trow + 4][16 * vt + tcol]);
    return u32x4_t{p[0], p[1], q2[0], q2[1]};
  };
  const int arow = 16 * wave + col;   // A-operand row of this lane
  // q rows (bf16) for the 4 key steps; A rows split for the 2 token steps
  u32x4_t qa[4], ah[2], al[2];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qa[ks] = ld16(&L.qs[arow][32 * ks + 8 * quad]);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const f32x4_t_ x0 = *reinterpret_cast<const f32x4_t_ *>(&L.A[arow][32 * ks + 8 * quad]);
    const f32x4_t_ x1 = *reinterpret_cast<const f32x4_t_ *>(&L.A[arow][32 * ks + 8 * quad + 4]);
    u32x2_t h0, l0, h1, l1;
    split4(x0, h0, l0);
    split4(x1, h1, l1);
    ah[ks] = u32x4_t{h0[0], h0[1], h1[0], h1[1]};
    al[ks] = u32x4_t{l0[0], l0[1], l1[0], l1[1]};
  }
  float eg[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) eg[j] = expf(L.sG[16 * wave + 4 * quad + j]);
  f32x4_t_ o[8];
#pragma unroll
  for (int vt = 0; vt < 8; ++vt) {
    f32x4_t_ a1 = {0.f, 0.f, 0.f, 0.f}, a2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      a1 = mfma16x32(qa[ks], bop(L.Sh, 32 * ks, vt), a1);
      a1 = mfma16x32(qa[ks], bop(L.Sl, 32 * ks, vt), a1);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x4_t dh = bop(L.Dh, 32 * ks, vt), dlo = bop(L.Dl, 32 * ks, vt);
      a2 = mfma16x32(ah[ks], dh, a2);
      a2 = mfma16x32(ah[ks], dlo, a2);
      a2 = mfma16x32(al[ks], dh, a2);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) o[vt][j] = eg[j] * a1[j] + a2[j];
  }
#pragma unroll
  for (int vt = 0; vt < 8; ++vt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * wave + 4 * quad + j;
      if (t < nval)
        out[int64_t(t0 + t) * o_t + h * o_h + 16 * vt + col] = bf16_t(f32_to_bf16_bits(o[vt][j]));
    }
}

bool rows_ok(const void *p, const int64_t *s) {
  return s[2] == 1 && s[0] % 8 == 0 && s[1] % 8 == 0 && wyh::aligned16(p);
}

}  // namespace

extern "C" int wy_gdn_chunk_prepare_wy(const void *k, const int64_t *ks, const void *v,
                                       const int64_t *vs, const float *beta, const int64_t *bs,
                                       const float *g, const int64_t *gs, float *w,
                                       float *u_base, float *g_cumsum, int token_num,
                                       int num_heads, int key_dim, int value_dim, void *stream) {
  if (!k || !ks || !v || !vs || !beta || !bs || !g || !gs || !w || !u_base || !g_cumsum)
    return WY_E_NULL;
  if (token_num <= 0 || num_heads <= 0) return WY_E_SHAPE;
  if (key_dim != kDK || value_dim != kDV) return WY_E_UNSUPPORTED;
  if (!rows_ok(k, ks) || !rows_ok(v, vs)) return WY_E_LAYOUT;
  const int N = (token_num + kC - 1) / kC;
  gdn_chunk_prepare_kernel<<<dim3(N, num_heads), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(k), ks[0], ks[1], static_cast<const bf16_t *>(v), vs[0], vs[1],
      beta, bs[0], bs[1], g, gs[0], gs[1], w, u_base, g_cumsum, token_num, num_heads);
  return wyh::launch_status();
}

extern "C" int wy_gdn_chunk_state(const void *k, const int64_t *ks, const float *w,
                                  const float *u_base, const float *g_cumsum, float *delta,
                                  float *chunk_state, float *final_state, int token_num,
                                  int num_heads, int key_dim, int value_dim, void *stream) {
  if (!k || !ks || !w || !u_base || !g_cumsum || !delta || !chunk_state || !final_state)
    return WY_E_NULL;
  if (token_num <= 0 || num_heads <= 0) return WY_E_SHAPE;
  if (key_dim != kDK || value_dim != kDV) return WY_E_UNSUPPORTED;
  if (!rows_ok(k, ks) || !wyh::aligned16(w)) return WY_E_LAYOUT;
  const int N = (token_num + kC - 1) / kC;
  // the attribute is per function: set once (a function-local static is
  // initialised exactly once, also under concurrent first calls)
  static const hipError_t lds_rc = hipFuncSetAttribute(
      reinterpret_cast<const void *>(&gdn_chunk_state_kernel),
      hipFuncAttributeMaxDynamicSharedMemorySize, kStateLds);
  if (lds_rc != hipSuccess) return int(lds_rc);
  gdn_chunk_state_kernel<<<dim3(num_heads, kDV / kBV), 512, kStateLds,
                           static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(k), ks[0], ks[1], w, u_base, g_cumsum, delta, chunk_state,
      final_state, token_num, num_heads, N);
  return wyh::launch_status();
}

extern "C" int wy_gdn_chunk_output(const void *q, const int64_t *qs, const void *k,
                                   const int64_t *ks, const float *delta, const float *g_cumsum,
                                   const float *chunk_state, void *out, const int64_t *os,
                                   int token_num, int num_heads, int key_dim, int value_dim,
                                   void *stream) {
  if (!q || !qs || !k || !ks || !delta || !g_cumsum || !chunk_state || !out || !os)
    return WY_E_NULL;
  if (token_num <= 0 || num_heads <= 0) return WY_E_SHAPE;
  if (key_dim != kDK || value_dim != kDV) return WY_E_UNSUPPORTED;
  if (!rows_ok(q, qs) || !rows_ok(k, ks) || os[2] != 1) return WY_E_LAYOUT;
  const int N = (token_num + kC - 1) / kC;
  static const hipError_t lds_rc = hipFuncSetAttribute(
      reinterpret_cast<const void *>(&gdn_chunk_output_kernel),
      hipFuncAttributeMaxDynamicSharedMemorySize, kOutLds);  // once, thread-safe
  if (lds_rc != hipSuccess) return int(lds_rc);
  gdn_chunk_output_kernel<<<dim3(N, num_heads), 256, kOutLds, static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(q), qs[0], qs[1], static_cast<const bf16_t *>(k), ks[0], ks[1],
      delta, g_cumsum, chunk_state, static_cast<bf16_t *>(out), os[0], os[1], token_num,
      num_heads);
  return wyh::launch_status();
}
