// Packed varlen causal GQA prefill attention on bf16 MFMA (gfx950).
//
// Workgroup = 4 wavefronts on one (sequence b, KV head h, 32-token query
// block).  Wave w owns query head 4h + w for those 32 tokens, so the four
// heads of the GQA group share every K/V tile the workgroup stages in LDS.
//
// Everything is computed transposed so that a lane owns one query row:
//   S^T = K Q^T   v_mfma_f32_32x32x16_bf16, A = K tile from LDS (token-major),
//                 B = q row (lane%32) held in registers for the whole kernel.
//                 C layout: lane l holds query row l%32 and 16 tokens
//                 8j + 4(l/32) + i of each 32-token slab.
//   O^T += V^T P^T  A = V^T from a transposed LDS tile, B = P^T taken straight
//                 from the S^T accumulators (no data movement): the k order of
//                 this contraction is the token permutation of the C layout,
//                 and the V^T operand is read in that same permutation.
// Row max / row sum are therefore lane-local plus one xor-32 exchange.
// Softmax in base 2 with the 1/sqrt(D) scale folded into log2(e); P is
// rounded to bf16 for the PV product as in the reference kernel
// (gqa_attention_varlen_causal.py:146-203).  K/V tiles of 64 tokens are
// prefetched into registers while the previous tile is consumed.
// Query blocks are launched heaviest first (LPT): blockIdx.z counts down.
#include "wy_common.h"

using namespace wy;

namespace {

constexpr int kD = 256;
constexpr int kG = 4;
constexpr int kBQ = 32;           // query tokens per workgroup
constexpr int kBN = 64;           // kv tokens per tile
constexpr int kKPitch = kD + 8;   // bf16 elements per K row in LDS (528 B)
constexpr int kVPitch = kBN + 4;  // bf16 elements per V^T row in LDS (136 B)
constexpr int kQBytes = kG * kBQ * kKPitch * 2;  // the four heads' query rows
constexpr int kLdsBytes = kQBytes + kBN * kKPitch * 2 + kD * kVPitch * 2;
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold (log2 units)

struct TileRegs {
  u32x4_t k[8];      // K rows: chunk u = tid + 256 j -> row u/32, dims (u%32)*8
  u32x4_t v[4][2];   // V token pairs: unit u = tid + 256 j -> pair u%32, dims (u/32)*8
};

// Rows past the sequence end are loaded from the last valid row (a safe
// address) and replaced by zeros with a select: no divergent branch around
// the loads, so they all stay in flight together.
__device__ __forceinline__ u32x4_t ld16_row_or_zero(const bf16_t *base, int64_t stride, int t,
                                                    int n, int c) {
  const int tc = t < n ? t : n - 1;
  const u32x4_t x = ld16(base + int64_t(tc) * stride + c);
  const u32x4_t z = {0u, 0u, 0u, 0u};
  return t < n ? x : z;
}

__device__ __forceinline__ void load_tile(TileRegs &r, const bf16_t *kseq, int64_t ks_t,
                                          const bf16_t *vseq, int64_t vs_t, int kv0,
                                          int n, int tid) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int u = tid + 256 * j;
    r.k[j] = ld16_row_or_zero(kseq, ks_t, kv0 + (u >> 5), n, (u & 31) * 8);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int u = tid + 256 * j;
    const int tp = u & 31, c = (u >> 5) * 8;
#pragma unroll
    for (int e = 0; e < 2; ++e) r.v[j][e] = ld16_row_or_zero(vseq, vs_t, kv0 + 2 * tp + e, n, c);
  }
}

__device__ __forceinline__ void store_tile(const TileRegs &r, bf16_t *sk, bf16_t *svt,
                                           int tid) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int u = tid + 256 * j;
    const int row = u >> 5, c = (u & 31) * 8;
    st16(sk + row * kKPitch + c, r.k[j]);
  }
  // V^T[d][t]: one 32-bit word = tokens (2tp, 2tp+1) of dim d.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int u = tid + 256 * j;
    const int tp = u & 31, c = (u >> 5) * 8;
    uint32_t *col = reinterpret_cast<uint32_t *>(svt + c * kVPitch + 2 * tp);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t a = r.v[j][0][w], b = r.v[j][1][w];
      // dim c+2w: low halves of (a, b); dim c+2w+1: high halves (v_perm_b32).
      col[(2 * w) * (kVPitch / 2)] = __builtin_amdgcn_perm(b, a, 0x05040100u);
      col[(2 * w + 1) * (kVPitch / 2)] = __builtin_amdgcn_perm(b, a, 0x07060302u);
    }
  }
}

__global__ __launch_bounds__(256) void varlen_causal_prefill_kernel(
    const bf16_t *__restrict__ q, int64_t qs_t, int64_t qs_h,
    const bf16_t *__restrict__ k, int64_t ks_t, int64_t ks_h,
    const bf16_t *__restrict__ v, int64_t vs_t, int64_t vs_h, bf16_t *__restrict__ out,
    int64_t os_t, int64_t os_h, const int32_t *__restrict__ cu, float qk_scale_log2) {
  extern __shared__ __align__(16) unsigned char smem[];
  bf16_t *sq = reinterpret_cast<bf16_t *>(smem);
  bf16_t *sk = sq + kG * kBQ * kKPitch;
  bf16_t *svt = sk + kBN * kKPitch;

  const int b = blockIdx.x, h = blockIdx.y;
  const int qb = gridDim.z - 1 - blockIdx.z;
  const int start = cu[b];
  const int n = cu[b + 1] - start;
  const int q0 = qb * kBQ;
  if (q0 >= n) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;     // k-group / row-quad selector of the MFMA layouts
  const int col = lane & 31;   // query row within the block
  const int hq = h * kG + wave;
  const int qrow = q0 + col;

  // The group's query rows (4 heads x 32 tokens) staged once in LDS; each
  // 16-dim k-step of S^T reads its B-operand slice from there, which keeps
  // the registers free for the accumulators and for read-ahead.
  {
    const bf16_t *qs = q + int64_t(start) * qs_t + h * kG * qs_h;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int u = tid + 256 * j;            // 4096 chunks of 16 bytes
      const int c = (u & 31) * 8, row = (u >> 5) & 31, hh = u >> 10;
      st16(sq + (hh * kBQ + row) * kKPitch + c,
           ld16_row_or_zero(qs + hh * qs_h, qs_t, q0 + row, n, c));
    }
  }
  const bf16_t *qrow_lds = sq + (wave * kBQ + col) * kKPitch + g * 8;

  f32x16_t o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
  float m_run = -INFINITY, l_part = 0.f;

  const bf16_t *kseq = k + int64_t(start) * ks_t + h * ks_h;
  const bf16_t *vseq = v + int64_t(start) * vs_t + h * vs_h;
  const int kv_end = min(q0 + kBQ, n);  // exclusive bound of keys any row can see
  const int n_tiles = (kv_end + kBN - 1) / kBN;

  TileRegs cur;
  load_tile(cur, kseq, ks_t, vseq, vs_t, 0, n, tid);
  for (int t = 0; t < n_tiles; ++t) {
    const int kv0 = t * kBN;
    __syncthreads();
    store_tile(cur, sk, svt, tid);
    __syncthreads();
    if (t + 1 < n_tiles) load_tile(cur, kseq, ks_t, vseq, vs_t, kv0 + kBN, n, tid);

    // ---- S^T for two 32-token slabs ----------------------------------------
    f32x16_t s[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[mt][e] = 0.f;
    }
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      const bf16x8_t qb = __builtin_bit_cast(bf16x8_t, ld16(qrow_lds + 16 * kk));
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const bf16_t *krow = sk + (mt * 32 + col) * kKPitch + g * 8;
        s[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, ld16(krow + 16 * kk)), qb, s[mt], 0, 0, 0);
      }
    }

    // ---- online softmax on the lane's row ------------------------------------
    const bool need_mask = kv0 + kBN > qrow - col || kv0 + kBN > n;  // uniform bound
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float x = s[mt][e] * qk_scale_log2;
        if (need_mask) {  // uniform branch; the per-element test is a select
          const int tok = kv0 + mt * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
          x = (tok > qrow || tok >= n) ? -INFINITY : x;
        }
        s[mt][e] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // Lazy rescaling: the running max moves only when the row max grows by
    // more than 2^8, so P <= 256 and the O/l rescale (a pass over 128
    // accumulators) is rare.  O/l is exact for any reference value m.
    const float m_new = fmaxf(m_run, mx);
    const bool grow = m_new > m_run + kRescaleLog2;
    const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
    if (grow) m_run = m_new;
    const float m_sub = m_run == -INFINITY ? 0.f : m_run;
    float psum = 0.f;
    u32x4_t pb[4];  // P^T B operands, k-steps 0..3 of the 64-token tile
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float a = __builtin_amdgcn_exp2f(s[mt][8 * kk + 2 * w] - m_sub);
          const float c = __builtin_amdgcn_exp2f(s[mt][8 * kk + 2 * w + 1] - m_sub);
          psum += a + c;
          pb[2 * mt + kk][w] = pack_bf16x2(a, c);
        }
    l_part = l_part * alpha + psum;
    if (__any(grow)) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
    }

    // ---- O^T += V^T P^T --------------------------------------------------------
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const bf16_t *vrow = svt + (dt * 32 + col) * kVPitch + 4 * g;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int t1 = 16 * ks;  // = 32*mt + 16*kk
        const u32x2_t lo = *reinterpret_cast<const u32x2_t *>(vrow + t1);
        const u32x2_t hi = *reinterpret_cast<const u32x2_t *>(vrow + t1 + 8);
        const u32x4_t a = {lo[0], lo[1], hi[0], hi[1]};
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                        __builtin_bit_cast(bf16x8_t, pb[ks]),
                                                        o[dt], 0, 0, 0);
      }
    }
  }

  // ---- normalise and store: lane holds row qrow, dims dt*32 + 8j + 4g + i -------
  const float l = l_part + __shfl_xor(l_part, 32);
  const float inv_l = 1.0f / l;
  if (qrow < n) {
    bf16_t *op = out + (int64_t(start) + qrow) * os_t + hq * os_h;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x2_t w = {pack_bf16x2(o[dt][4 * j] * inv_l, o[dt][4 * j + 1] * inv_l),
                           pack_bf16x2(o[dt][4 * j + 2] * inv_l, o[dt][4 * j + 3] * inv_l)};
        *reinterpret_cast<u32x2_t *>(op + dt * 32 + 8 * j + 4 * g) = w;
      }
  }
}

}  // namespace

extern "C" int wy_varlen_causal_prefill(const void *q, const int64_t *qs, const void *k,
                                        const int64_t *ks, const void *v,
                                        const int64_t *vs, void *out, const int64_t *os,
                                        const int32_t *cu_seqlens, int batch,
                                        int num_q_heads, int num_kv_heads, int head_dim,
                                        int max_seqlen, void *stream) {
  if (!q || !qs || !k || !ks || !v || !vs || !out || !os || !cu_seqlens) return WY_E_NULL;
  if (batch < 0 || num_kv_heads <= 0 || max_seqlen < 0) return WY_E_SHAPE;
  if (head_dim != kD || num_q_heads != kG * num_kv_heads) return WY_E_UNSUPPORTED;
  if (qs[2] != 1 || ks[2] != 1 || vs[2] != 1 || os[2] != 1 || qs[0] % 8 || qs[1] % 8 ||
      ks[0] % 8 || ks[1] % 8 || vs[0] % 8 || vs[1] % 8 || os[0] % 4 || os[1] % 4 ||
      !wyh::aligned16(q) || !wyh::aligned16(k) || !wyh::aligned16(v) ||
      (reinterpret_cast<uintptr_t>(out) & 7u))
    return WY_E_LAYOUT;
  if (batch == 0 || max_seqlen == 0) return WY_OK;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&varlen_causal_prefill_kernel),
        hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return int(e);
    attr_set = true;
  }
  dim3 grid(batch, num_kv_heads, (max_seqlen + kBQ - 1) / kBQ);
  varlen_causal_prefill_kernel<<<grid, 256, kLdsBytes, static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(q), qs[0], qs[1], static_cast<const bf16_t *>(k), ks[0],
      ks[1], static_cast<const bf16_t *>(v), vs[0], vs[1], static_cast<bf16_t *>(out),
      os[0], os[1], cu_seqlens, kLog2e / sqrtf(float(head_dim)));
  return wyh::launch_status();
}
