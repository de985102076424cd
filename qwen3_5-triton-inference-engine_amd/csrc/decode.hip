// Paged GQA decode attention, split-K over 16-token pages (gfx950).
//
// Partial pass: one 256-thread workgroup per (sequence b, KV head h, split s).
// The split's pages are dealt round-robin to the four wavefronts; each wave
// keeps its own online-softmax state for the 4 query heads of the KV group, so
// one read of a K/V page serves all 4 heads.  Per page and wave:
//   * K (16 tokens x 256 dims) is loaded straight into the B operand of
//     v_mfma_f32_16x16x32_bf16 -- lane (token n = l%16, dim group g = l/16)
//     reads 16 bytes at dims 32i + 8g, so each instruction reads sixteen
//     64-byte row segments; q (4 heads, rows 4..15 zero) is the A operand and
//     8 MFMAs give the 4 x 16 score tile in lanes 0..15.
//   * V is read row-contiguous (lane l: token 2i + l/32, dims (l%32)*8..+8)
//     and P.V runs on the VALU in fp32 with P rounded to bf16, the rounding
//     the reference applies before its PV dot.
//   * The softmax max/sum reduce across the 16 token lanes with xor shuffles.
// After the page loop the four wave states merge through LDS and one fp32
// (m, l, acc) triple per query head is written for the split.
//
// Merge pass: one wavefront per (b, query head) folds the active splits with
// exp(m_s - max m) weights and writes bf16.
//
// Split partition (both passes compute it from pos on the device, so the grid
// is static and the pair is graph-safe):
//   npg = ceil((pos+1)/16), pps = max(ceil(npg/128), min_pps),
//   split s covers pages [s*pps, min((s+1)*pps, npg)), active = ceil(npg/pps).
// With min_pps = 1 this is exactly the reference partition
// (gqa_attention_decode_paged.py:675-682, 779-784); a larger min_pps trades
// split count for less fp32 scratch traffic.
#include "wy_common.h"

using namespace wy;

namespace {

constexpr int kD = 256;   // head_dim
constexpr int kG = 4;     // query heads per KV head
constexpr int kWaves = 4; // wavefronts per workgroup

__device__ __forceinline__ int split_pps(int npg, int min_pps) {
  const int p = (npg + kMaxSplits - 1) / kMaxSplits;
  return p > min_pps ? p : min_pps;
}

__device__ __forceinline__ float readlane0(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// Max / sum over the 16 lanes of each row of 16 (lanes 0..15 hold the scores).
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, __shfl_xor(v, 1));
  v = fmaxf(v, __shfl_xor(v, 2));
  v = fmaxf(v, __shfl_xor(v, 4));
  v = fmaxf(v, __shfl_xor(v, 8));
  return v;
}
__device__ __forceinline__ float sum16(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  return v;
}

struct PageRegs {
  u32x4_t k[8];  // MFMA B operand, one per 32-dim step
  u32x4_t v[8];  // row-contiguous V, tokens 2i + lane/32
};

__device__ __forceinline__ void load_page(PageRegs &r, const bf16_t *kbase,
                                          const bf16_t *vbase, int64_t kc_s,
                                          int64_t vc_s, int lane) {
  const bf16_t *kp = kbase + (lane & 15) * kc_s + (lane >> 4) * 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) r.k[i] = ld16(kp + 32 * i);
  const bf16_t *vp = vbase + (lane >> 5) * vc_s + (lane & 31) * 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) r.v[i] = ld16(vp + 2 * i * vc_s);
}

__global__ __launch_bounds__(256) void paged_decode_split_kernel(
    const bf16_t *__restrict__ q, int64_t qs_b, int64_t qs_h, int64_t qs_d,
    const bf16_t *__restrict__ kc, const bf16_t *__restrict__ vc, int64_t kc_p,
    int64_t kc_h, int64_t kc_s, int64_t vc_p, int64_t vc_h, int64_t vc_s,
    const int32_t *__restrict__ bt, int64_t bt_b, const int64_t *__restrict__ pos,
    float *__restrict__ mp, float *__restrict__ lp, float *__restrict__ ap,
    int64_t ml_b, int64_t ml_h, int64_t ml_s, int64_t a_b, int64_t a_h, int64_t a_s,
    float scale, int min_pps) {
  __shared__ float4 sm_p[kWaves][kPage];          // bf16-rounded P, [token][head]
  __shared__ float sm_ml[kWaves][2][kG];          // per-wave m, l
  __shared__ float4 sm_acc[kWaves][kG][kD / 4];   // per-wave unnormalised acc

  const int b = blockIdx.x, h = blockIdx.y, s = blockIdx.z;
  const int seq_len = int(pos[b]) + 1;
  const int npg = (seq_len + kPage - 1) / kPage;
  const int pps = split_pps(npg, min_pps);
  const int p0 = s * pps;
  if (p0 >= npg) return;  // inactive split: uniform over the workgroup
  const int p1 = min(p0 + pps, npg);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // q rows of the group as the MFMA A operand (rows 4..15 are zero).
  bf16x8_t qa[8];
  {
    const int row = lane & 15, g = lane >> 4;
    const bf16_t *qrow = q + b * qs_b + (h * kG + (row & 3)) * qs_h;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      u32x4_t w = {0u, 0u, 0u, 0u};
      if (row < kG) {
        const int d0 = 32 * i + 8 * g;
        if (qs_d == 1) {
          w = ld16(qrow + d0);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            w[e] = uint32_t(qrow[(d0 + 2 * e) * qs_d]) |
                   (uint32_t(qrow[(d0 + 2 * e + 1) * qs_d]) << 16);
        }
      }
      qa[i] = __builtin_bit_cast(bf16x8_t, w);
    }
  }

  float m_run[kG], l_run[kG], acc[kG][8];
#pragma unroll
  for (int r = 0; r < kG; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;
  }

  const bf16_t *kh = kc + h * kc_h;
  const bf16_t *vh = vc + h * vc_h;
  const int32_t *btrow = bt + b * bt_b;

  int p = p0 + wave;
  PageRegs cur;
  if (p < p1) {
    const int64_t phys = btrow[p];
    load_page(cur, kh + phys * kc_p, vh + phys * vc_p, kc_s, vc_s, lane);
  }
  for (; p < p1; p += kWaves) {
    PageRegs nxt;
    const int pn = p + kWaves;
    if (pn < p1) {
      const int64_t physn = btrow[pn];
      load_page(nxt, kh + physn * kc_p, vh + physn * vc_p, kc_s, vc_s, lane);
    }

    // ---- scores: 4 heads x 16 tokens in lanes 0..15 ------------------------
    f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i)
      sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          qa[i], __builtin_bit_cast(bf16x8_t, cur.k[i]), sc, 0, 0, 0);
    const bool valid = p * kPage + (lane & 15) < seq_len;
    float pr[kG], alpha[kG];
#pragma unroll
    for (int r = 0; r < kG; ++r) {
      const float x = valid ? sc[r] * scale : -INFINITY;
      const float mx = readlane0(max16(x));
      const float m_new = fmaxf(m_run[r], mx);
      alpha[r] = __expf(m_run[r] - m_new);
      pr[r] = __expf(x - m_new);
      const float ps = readlane0(sum16(pr[r]));
      l_run[r] = l_run[r] * alpha[r] + ps;
      m_run[r] = m_new;
    }
    if (lane < kPage)
      sm_p[wave][lane] = make_float4(round_bf16(pr[0]), round_bf16(pr[1]),
                                     round_bf16(pr[2]), round_bf16(pr[3]));
    __builtin_amdgcn_wave_barrier();

    // Rows past the sequence end in the last page may hold anything (even NaN):
    // zero them so 0 * garbage cannot reach the accumulator.
    if ((p + 1) * kPage > seq_len) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (p * kPage + 2 * i + (lane >> 5) >= seq_len) cur.v[i] = u32x4_t{0u, 0u, 0u, 0u};
    }
    // ---- acc = acc * alpha + P V (lane: dims (lane%32)*8.., tokens of parity lane/32)
#pragma unroll
    for (int r = 0; r < kG; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[r][e] *= alpha[r];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 pv = sm_p[wave][2 * i + (lane >> 5)];
      const float pw[kG] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float v0 = bf16_lo(cur.v[i][w]), v1 = bf16_hi(cur.v[i][w]);
#pragma unroll
        for (int r = 0; r < kG; ++r) {
          acc[r][2 * w] = fmaf(pw[r], v0, acc[r][2 * w]);
          acc[r][2 * w + 1] = fmaf(pw[r], v1, acc[r][2 * w + 1]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    if (pn < p1) cur = nxt;
  }

  // ---- fold the two token parities, then the four waves ---------------------
#pragma unroll
  for (int r = 0; r < kG; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] += __shfl_xor(acc[r][e], 32);
  if (lane < 32) {
#pragma unroll
    for (int r = 0; r < kG; ++r) {
      sm_acc[wave][r][lane * 2] = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
      sm_acc[wave][r][lane * 2 + 1] =
          make_float4(acc[r][4], acc[r][5], acc[r][6], acc[r][7]);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < kG; ++r) {
      sm_ml[wave][0][r] = m_run[r];
      sm_ml[wave][1][r] = l_run[r];
    }
  }
  __syncthreads();

  const int r = threadIdx.x >> 6;  // query head within the group
  const int c4 = threadIdx.x & 63; // float4 column
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_ml[w][0][r]);
  float L = 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float a = __expf(sm_ml[w][0][r] - M);
    L += a * sm_ml[w][1][r];
    const float4 x = sm_acc[w][r][c4];
    A.x += a * x.x;
    A.y += a * x.y;
    A.z += a * x.z;
    A.w += a * x.w;
  }
  const int hq = h * kG + r;
  *reinterpret_cast<float4 *>(ap + b * a_b + hq * a_h + s * a_s + c4 * 4) = A;
  if (c4 == 0) {
    mp[b * ml_b + hq * ml_h + s * ml_s] = M;
    lp[b * ml_b + hq * ml_h + s * ml_s] = L;
  }
}

// One wavefront per (sequence, query head); lane owns 4 of the 256 dims.
__global__ __launch_bounds__(64) void paged_decode_combine_kernel(
    const float *__restrict__ mp, const float *__restrict__ lp,
    const float *__restrict__ ap, int64_t ml_b, int64_t ml_h, int64_t ml_s,
    int64_t a_b, int64_t a_h, int64_t a_s, const int64_t *__restrict__ pos,
    bf16_t *__restrict__ out, int64_t o_b, int64_t o_h, int64_t o_d, int min_pps) {
  const int b = blockIdx.x, hq = blockIdx.y, lane = threadIdx.x;
  const int seq_len = int(pos[b]) + 1;
  const int npg = (seq_len + kPage - 1) / kPage;
  const int pps = split_pps(npg, min_pps);
  const int nact = (npg + pps - 1) / pps;
  const float *mrow = mp + b * ml_b + hq * ml_h;
  const float *lrow = lp + b * ml_b + hq * ml_h;
  const float *arow = ap + b * a_b + hq * a_h + lane * 4;

  float mx = -INFINITY;
  for (int s = lane; s < nact; s += 64) mx = fmaxf(mx, mrow[s * ml_s]);
  mx = wave_max(mx);

  float L = 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  int s = 0;
  for (; s + 4 <= nact; s += 4) {
    float4 x[4];
    float a[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      x[u] = *reinterpret_cast<const float4 *>(arow + (s + u) * a_s);
      a[u] = __expf(mrow[(s + u) * ml_s] - mx);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      L += a[u] * lrow[(s + u) * ml_s];
      A.x += a[u] * x[u].x;
      A.y += a[u] * x[u].y;
      A.z += a[u] * x[u].z;
      A.w += a[u] * x[u].w;
    }
  }
  for (; s < nact; ++s) {
    const float4 x = *reinterpret_cast<const float4 *>(arow + s * a_s);
    const float a = __expf(mrow[s * ml_s] - mx);
    L += a * lrow[s * ml_s];
    A.x += a * x.x;
    A.y += a * x.y;
    A.z += a * x.z;
    A.w += a * x.w;
  }
  bf16_t *orow = out + b * o_b + hq * o_h;
  const int d = lane * 4;
  if (o_d == 1) {
    u32x2_t w = {pack_bf16x2(A.x / L, A.y / L), pack_bf16x2(A.z / L, A.w / L)};
    *reinterpret_cast<u32x2_t *>(orow + d) = w;
  } else {
    orow[(d + 0) * o_d] = bf16_t(f32_to_bf16_bits(A.x / L));
    orow[(d + 1) * o_d] = bf16_t(f32_to_bf16_bits(A.y / L));
    orow[(d + 2) * o_d] = bf16_t(f32_to_bf16_bits(A.z / L));
    orow[(d + 3) * o_d] = bf16_t(f32_to_bf16_bits(A.w / L));
  }
}

}  // namespace

extern "C" int wy_paged_decode_split(const void *q, const int64_t *qs, const void *k_cache,
                                     const void *v_cache, const int64_t *kcs,
                                     const int64_t *vcs, const int32_t *block_table,
                                     int64_t bt_stride0, const int64_t *pos,
                                     float *m_partial, float *l_partial,
                                     float *acc_partial, const int64_t *mls,
                                     const int64_t *as, int batch, int num_q_heads,
                                     int num_kv_heads, int head_dim, int max_pages,
                                     int min_pages_per_split, void *stream) {
  if (!q || !qs || !k_cache || !v_cache || !kcs || !vcs || !block_table || !pos ||
      !m_partial || !l_partial || !acc_partial || !mls || !as)
    return WY_E_NULL;
  if (batch < 0 || num_kv_heads <= 0 || max_pages <= 0 || min_pages_per_split <= 0)
    return WY_E_SHAPE;
  if (head_dim != kD || num_q_heads != kG * num_kv_heads) return WY_E_UNSUPPORTED;
  if (kcs[3] != 1 || vcs[3] != 1 || kcs[2] % 8 || vcs[2] % 8 || kcs[1] % 8 ||
      vcs[1] % 8 || kcs[0] % 8 || vcs[0] % 8 || as[3] != 1 || as[2] % 4 ||
      as[1] % 4 || as[0] % 4 || !wyh::aligned16(k_cache) || !wyh::aligned16(v_cache) ||
      !wyh::aligned16(acc_partial) ||
      (qs[2] == 1 && (qs[0] % 8 || qs[1] % 8 || !wyh::aligned16(q))))
    return WY_E_LAYOUT;
  if (batch == 0) return WY_OK;
  int splits = (max_pages + min_pages_per_split - 1) / min_pages_per_split;
  if (splits > kMaxSplits) splits = kMaxSplits;
  dim3 grid(batch, num_kv_heads, splits);
  paged_decode_split_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(q), qs[0], qs[1], qs[2],
      static_cast<const bf16_t *>(k_cache), static_cast<const bf16_t *>(v_cache), kcs[0],
      kcs[1], kcs[2], vcs[0], vcs[1], vcs[2], block_table, bt_stride0, pos, m_partial,
      l_partial, acc_partial, mls[0], mls[1], mls[2], as[0], as[1], as[2],
      1.0f / sqrtf(float(head_dim)), min_pages_per_split);
  return wyh::launch_status();
}

extern "C" int wy_paged_decode_combine(const float *m_partial, const float *l_partial,
                                       const float *acc_partial, const int64_t *mls,
                                       const int64_t *as, const int64_t *pos, void *out,
                                       const int64_t *os, int batch, int num_q_heads,
                                       int head_dim, int min_pages_per_split,
                                       void *stream) {
  if (!m_partial || !l_partial || !acc_partial || !mls || !as || !pos || !out || !os)
    return WY_E_NULL;
  if (batch < 0 || num_q_heads <= 0 || min_pages_per_split <= 0) return WY_E_SHAPE;
  if (head_dim != kD) return WY_E_UNSUPPORTED;
  if (as[3] != 1 || as[2] % 4 || as[1] % 4 || as[0] % 4 || !wyh::aligned16(acc_partial) ||
      (os[2] == 1 && (os[0] % 4 || os[1] % 4 ||
                      (reinterpret_cast<uintptr_t>(out) & 7u))))
    return WY_E_LAYOUT;
  if (batch == 0) return WY_OK;
  dim3 grid(batch, num_q_heads);
  paged_decode_combine_kernel<<<grid, 64, 0, static_cast<hipStream_t>(stream)>>>(
      m_partial, l_partial, acc_partial, mls[0], mls[1], mls[2], as[0], as[1], as[2], pos,
      static_cast<bf16_t *>(out), os[0], os[1], os[2], min_pages_per_split);
  return wyh::launch_status();
}
