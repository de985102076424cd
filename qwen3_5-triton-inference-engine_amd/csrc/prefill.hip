// Packed varlen causal GQA prefill attention on bf16 MFMA (gfx950).
//
// Two launches:
//   1. vt_pack: V [total, H_kv, D] -> V^T workspace [H_kv, D, T_pad], each
//      sequence's tokens at a 64-aligned offset pstart(b) = 64*(ceil(cu[b]/64)+b)
//      and zero-filled up to the next multiple of 64.  This moves the
//      transposition the PV product needs out of the attention loop.
//   2. the attention kernel: one workgroup = 4 wavefronts on (sequence b,
//      KV head h, 32-token query block); wave w owns query head 4h + w, so
//      the four heads of the GQA group share every K/V tile in LDS.
//
// Attention is computed transposed so that a lane owns one query row:
//   S^T = K Q^T      v_mfma_f32_32x32x16_bf16; A = K tile (LDS), B = q row
//                    (lane%32) kept in registers for the whole kernel.
//   O^T += V^T P^T   A = V^T tile (LDS), B = P^T taken straight from the S^T
//                    accumulators.
// The K tile's LDS rows are a permutation of the 64 tokens, chosen so that
// the S^T accumulator registers of lane (col, g) hold tokens 32mt + 16g + r
// (r = register index 0..15): every PV k-step then reads 8 contiguous tokens
// of V^T, one 16-byte LDS read.  Row max / sum are lane-local plus one xor-32
// exchange.  Softmax in base 2 with 1/sqrt(D) folded into log2(e); P is
// rounded to bf16 for PV as in the reference kernel
// (gqa_attention_varlen_causal.py:146-203); the running max is moved lazily
// (only when a row max grows by more than 2^8), exact after the final 1/l.
//
// K and V^T tiles travel global -> LDS with global_load_lds_dwordx4 (no
// registers), double-buffered: tile t+1 is in flight while tile t is
// consumed, one barrier per tile.  LDS rows are XOR-swizzled by 16-byte
// chunk (chunk ^ (row & 7)) so the MFMA operand reads are conflict-free.
// Rows past a sequence's end are loaded from its last row (a safe address)
// and masked in the scores; V^T past the end is zero from the pre-pass.
// Query blocks are launched heaviest first (LPT): blockIdx.z counts down.
#include "wy_common.h"

using namespace wy;

namespace {

constexpr int kD = 256;
constexpr int kG = 4;
constexpr int kBQ = 32;                  // query tokens per workgroup
constexpr int kBN = 64;                  // kv tokens per tile
constexpr int kTileK = kBN * kD * 2;     // bytes of one K tile  (32 KiB)
constexpr int kTileV = kD * kBN * 2;     // bytes of one V^T tile (32 KiB)
constexpr int kStage = kTileK + kTileV;  // one pipeline stage
constexpr int kLdsBytes = 2 * kStage;    // double buffered: 128 KiB
constexpr float kRescaleLog2 = 8.0f;     // lazy-rescale threshold (log2 units)

typedef __attribute__((address_space(3))) void lds_void_t;
typedef const __attribute__((address_space(1))) void gbl_void_t;

__device__ __forceinline__ int64_t pstart(int cu_b, int b) {
  return 64 * (int64_t((cu_b + 63) >> 6) + b);
}

// Token held by LDS row `row` of a K tile (see the header comment).
__device__ __forceinline__ int k_row_token(int row) {
  const int mt = row >> 5, r = row & 31;
  return 32 * mt + 16 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3);
}

__device__ __forceinline__ void lds_dma16(const void *src, unsigned char *lds_dst) {
  __builtin_amdgcn_global_load_lds((gbl_void_t *)(src),
                                   (lds_void_t *)(lds_dst), 16, 0, 0);
}

// ------------------------------------------------------------------ V^T pack
__global__ __launch_bounds__(256) void vt_pack_kernel(const bf16_t *__restrict__ v,
                                                      int64_t vs_t, int64_t vs_h,
                                                      bf16_t *__restrict__ vt, int64_t t_pad,
                                                      const int32_t *__restrict__ cu) {
  __shared__ bf16_t tile[kBN][kD + 2];
  const int b = blockIdx.z, h = blockIdx.y, t0 = blockIdx.x * kBN;
  const int start = cu[b], n = cu[b + 1] - start;
  if (t0 >= n) return;
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int u = tid + 256 * j;
    const int row = u >> 5, c = (u & 31) * 8;
    const int t = t0 + row;
    const int tc = t < n ? t : n - 1;
    u32x4_t x = ld16(v + (int64_t(start) + tc) * vs_t + h * vs_h + c);
    if (t >= n) x = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      *reinterpret_cast<uint32_t *>(&tile[row][c + 2 * w]) = x[w];
    }
  }
  __syncthreads();
  bf16_t *dst = vt + int64_t(h) * kD * t_pad + pstart(start, b) + t0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int u = tid + 256 * j;
    const int dim = u >> 3, tc = (u & 7) * 8;
    u32x4_t w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = uint32_t(tile[tc + 2 * e][dim]) | (uint32_t(tile[tc + 2 * e + 1][dim]) << 16);
    st16(dst + int64_t(dim) * t_pad + tc, w);
  }
}

// ------------------------------------------------------------------ attention
__global__ __launch_bounds__(256) void varlen_causal_prefill_kernel(
    const bf16_t *__restrict__ q, int64_t qs_t, int64_t qs_h,
    const bf16_t *__restrict__ k, int64_t ks_t, int64_t ks_h,
    const bf16_t *__restrict__ vt, int64_t t_pad, bf16_t *__restrict__ out, int64_t os_t,
    int64_t os_h, const int32_t *__restrict__ cu, float qk_scale_log2) {
  extern __shared__ __align__(16) unsigned char smem[];

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

  const bf16_t *kseq = k + int64_t(start) * ks_t + h * ks_h;
  const bf16_t *vtseq = vt + int64_t(h) * kD * t_pad + pstart(start, b);
  const int kv_end = min(q0 + kBQ, n);  // exclusive bound of keys any row can see
  const int n_tiles = (kv_end + kBN - 1) / kBN;

  // Issue one tile's K and V^T (64 KiB) into stage `st`: 64 wave-wide 1 KiB
  // DMA instructions, 16 per wave.
  auto issue_tile = [&](int t, int st) {
    unsigned char *sk = smem + st * kStage;
    unsigned char *sv = sk + kTileK;
    const int kv0 = t * kBN;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int blk = wave * 8 + i;          // 1 KiB block = K rows 2blk, 2blk+1
      const int row = 2 * blk + (lane >> 5);
      const int c = (lane & 31) ^ (row & 7); // global chunk stored at LDS chunk lane&31
      int tok = kv0 + k_row_token(row);
      tok = tok < n ? tok : n - 1;
      lds_dma16(kseq + int64_t(tok) * ks_t + c * 8, sk + blk * 1024);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int blk = wave * 8 + i;          // 1 KiB block = V^T rows 8blk .. 8blk+7
      const int dim = 8 * blk + (lane >> 3);
      const int c = (lane & 7) ^ (dim & 7);
      lds_dma16(vtseq + int64_t(dim) * t_pad + kv0 + c * 8, sv + blk * 1024);
    }
  };

  issue_tile(0, 0);

  // q row as the B operand of S^T, one 16-byte slice per 16-dim k-step.
  bf16x8_t qb_op[16];
  {
    const int qc = qrow < n ? qrow : n - 1;
    const bf16_t *qp = q + (int64_t(start) + qc) * qs_t + hq * qs_h + g * 8;
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      u32x4_t x = ld16(qp + 16 * kk);
      if (qrow >= n) x = u32x4_t{0u, 0u, 0u, 0u};
      qb_op[kk] = __builtin_bit_cast(bf16x8_t, x);
    }
  }

  f32x16_t o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
  float m_run = -INFINITY, l_part = 0.f;

  for (int t = 0; t < n_tiles; ++t) {
    const int kv0 = t * kBN;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's DMA for tile t
    __syncthreads();  // all of tile t landed; everyone is done with tile t-1
    if (t + 1 < n_tiles) issue_tile(t + 1, (t + 1) & 1);
    const unsigned char *sk = smem + (t & 1) * kStage;
    const unsigned char *sv = sk + kTileK;

    // ---- S^T for two 32-row slabs of the K tile -----------------------------
    f32x16_t s[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int e = 0; e < 16; ++e) s[mt][e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int row = mt * 32 + col;
        const u32x4_t a = ld16(sk + row * (kD * 2) + (((2 * kk + g) ^ (row & 7)) << 4));
        s[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                        qb_op[kk], s[mt], 0, 0, 0);
      }
    }

    // ---- online softmax on the lane's row ------------------------------------
    // register r of slab mt holds token kv0 + 32mt + 16g + r
    const bool need_mask = kv0 + kBN > q0 || kv0 + kBN > n;  // uniform
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float x = s[mt][e] * qk_scale_log2;
        if (need_mask) {
          const int tok = kv0 + 32 * mt + 16 * g + e;
          x = (tok > qrow || tok >= n) ? -INFINITY : x;
        }
        s[mt][e] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const bool grow = m_new > m_run + kRescaleLog2;
    const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
    if (grow) m_run = m_new;
    const float m_sub = m_run == -INFINITY ? 0.f : m_run;
    float psum = 0.f;
    u32x4_t pb[4];  // P^T B operands: k-step 2mt+kk = tokens 32mt+16g+8kk .. +7
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

    // ---- O^T += V^T P^T ------------------------------------------------------
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int dim = dt * 32 + col;
      const unsigned char *vrow = sv + dim * (kBN * 2);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int chunk = 4 * (ks >> 1) + 2 * g + (ks & 1);
        const u32x4_t a = ld16(vrow + ((chunk ^ (dim & 7)) << 4));
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

int64_t t_pad_for(int64_t total_tokens, int batch) {
  return 64 * ((total_tokens + 63) / 64 + batch) + 64;
}

}  // namespace

extern "C" size_t wy_varlen_causal_prefill_workspace_size(int64_t total_tokens, int batch,
                                                          int num_kv_heads, int head_dim) {
  if (total_tokens < 0 || batch < 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
  return size_t(num_kv_heads) * size_t(head_dim) * size_t(t_pad_for(total_tokens, batch)) * 2;
}

extern "C" int wy_varlen_causal_prefill(const void *q, const int64_t *qs, const void *k,
                                        const int64_t *ks, const void *v,
                                        const int64_t *vs, void *out, const int64_t *os,
                                        const int32_t *cu_seqlens, int batch,
                                        int num_q_heads, int num_kv_heads, int head_dim,
                                        int max_seqlen, int64_t total_tokens, void *workspace,
                                        size_t workspace_bytes, void *stream) {
  if (!q || !qs || !k || !ks || !v || !vs || !out || !os || !cu_seqlens || !workspace)
    return WY_E_NULL;
  if (batch < 0 || num_kv_heads <= 0 || max_seqlen < 0 || total_tokens < 0)
    return WY_E_SHAPE;
  if (head_dim != kD || num_q_heads != kG * num_kv_heads) return WY_E_UNSUPPORTED;
  if (qs[2] != 1 || ks[2] != 1 || vs[2] != 1 || os[2] != 1 || qs[0] % 8 || qs[1] % 8 ||
      ks[0] % 8 || ks[1] % 8 || vs[0] % 8 || vs[1] % 8 || os[0] % 4 || os[1] % 4 ||
      !wyh::aligned16(q) || !wyh::aligned16(k) || !wyh::aligned16(v) ||
      !wyh::aligned16(workspace) || (reinterpret_cast<uintptr_t>(out) & 7u))
    return WY_E_LAYOUT;
  if (workspace_bytes <
      wy_varlen_causal_prefill_workspace_size(total_tokens, batch, num_kv_heads, head_dim))
    return WY_E_SHAPE;
  if (batch == 0 || max_seqlen == 0) return WY_OK;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&varlen_causal_prefill_kernel),
        hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return int(e);
    attr_set = true;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t t_pad = t_pad_for(total_tokens, batch);
  bf16_t *vt = static_cast<bf16_t *>(workspace);
  dim3 pgrid((max_seqlen + kBN - 1) / kBN, num_kv_heads, batch);
  vt_pack_kernel<<<pgrid, 256, 0, s>>>(static_cast<const bf16_t *>(v), vs[0], vs[1], vt, t_pad,
                                      cu_seqlens);
  dim3 grid(batch, num_kv_heads, (max_seqlen + kBQ - 1) / kBQ);
  varlen_causal_prefill_kernel<<<grid, 256, kLdsBytes, s>>>(
      static_cast<const bf16_t *>(q), qs[0], qs[1], static_cast<const bf16_t *>(k), ks[0],
      ks[1], vt, t_pad, static_cast<bf16_t *>(out), os[0], os[1], cu_seqlens,
      kLog2e / sqrtf(float(head_dim)));
  return wyh::launch_status();
}
