// Page-pool writers: the per-step K/V append and the packed varlen scatter.
//
// Both are pure data movement, bit-exact by construction.  The address of a
// token row in the pool follows the page-table contract of
// engine/paging.py:23 (reference):
//     row(t, h) = (block_table[t // 16] * H + h) * 16 + t % 16
// expressed here through the pool's four strides so any pool layout with a
// unit innermost stride takes the 16-byte path.
#include "wy_common.h"

using namespace wy;

namespace {

// ---------------------------------------------------------------- append --
// One 64-lane wavefront per (sequence, KV head); lanes move 16-byte chunks of
// the K row and then the V row.  Reference: gqa_attention_decode_paged.py:176-250.
template <bool kVec>
__global__ __launch_bounds__(64) void paged_kv_append_kernel(
    bf16_t *__restrict__ kc, bf16_t *__restrict__ vc, int64_t kc_p, int64_t kc_h,
    int64_t kc_s, int64_t kc_d, int64_t vc_p, int64_t vc_h, int64_t vc_s,
    int64_t vc_d, const bf16_t *__restrict__ kn, const bf16_t *__restrict__ vn,
    int64_t kn_b, int64_t kn_h, int64_t kn_d, int64_t vn_b, int64_t vn_h,
    int64_t vn_d, const int32_t *__restrict__ bt, int64_t bt_b,
    const int64_t *__restrict__ pos, int D) {
  const int b = blockIdx.x, h = blockIdx.y;
  const int64_t p = pos[b];
  const int64_t lp = p / kPage, slot = p % kPage;
  const int64_t phys = int64_t(bt[b * bt_b + lp]);
  bf16_t *kdst = kc + phys * kc_p + h * kc_h + slot * kc_s;
  bf16_t *vdst = vc + phys * vc_p + h * vc_h + slot * vc_s;
  const bf16_t *ksrc = kn + b * kn_b + h * kn_h;
  const bf16_t *vsrc = vn + b * vn_b + h * vn_h;
  if constexpr (kVec) {
    const int chunks = D / 8;
    for (int i = threadIdx.x; i < 2 * chunks; i += 64) {
      if (i < chunks)
        st16(kdst + i * 8, ld16(ksrc + i * 8));
      else
        st16(vdst + (i - chunks) * 8, ld16(vsrc + (i - chunks) * 8));
    }
  } else {
    for (int d = threadIdx.x; d < D; d += 64) {
      kdst[d * kc_d] = ksrc[d * kn_d];
      vdst[d * vc_d] = vsrc[d * vn_d];
    }
  }
}

// ----------------------------------------------------------- varlen fill --
// One 256-thread workgroup per (logical page, KV head, sequence): it moves the
// page's valid rows of K and V (at most 16 x D each).  Pages past the
// sequence's length exit at once.  Rows past the sequence end inside the last
// page are neither read nor written.
// Reference: gqa_attention_decode_paged.py:398-489.
template <bool kVec>
__global__ __launch_bounds__(256) void paged_kv_fill_varlen_kernel(
    bf16_t *__restrict__ kc, bf16_t *__restrict__ vc, int64_t kc_p, int64_t kc_h,
    int64_t kc_s, int64_t kc_d, int64_t vc_p, int64_t vc_h, int64_t vc_s,
    int64_t vc_d, const bf16_t *__restrict__ k, const bf16_t *__restrict__ v,
    int64_t k_h, int64_t k_t, int64_t k_d, int64_t v_h, int64_t v_t, int64_t v_d,
    const int32_t *__restrict__ bt, int64_t bt_b, const int32_t *__restrict__ cu,
    int D) {
  const int lp = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int start = cu[b];
  const int n = cu[b + 1] - start;
  const int t0 = lp * kPage;
  if (t0 >= n) return;
  const int rows = min(kPage, n - t0);
  const int64_t phys = int64_t(bt[b * bt_b + lp]);
  bf16_t *kdst = kc + phys * kc_p + h * kc_h;
  bf16_t *vdst = vc + phys * vc_p + h * vc_h;
  const int64_t tok0 = int64_t(start) + t0;
  const bf16_t *ksrc = k + h * k_h + tok0 * k_t;
  const bf16_t *vsrc = v + h * v_h + tok0 * v_t;
  if constexpr (kVec) {
    // Each thread requests its K and V chunks of a round (two of each)
    // before it stores any: one memory round trip per round instead of one
    // per chunk (a full page of D = 256 is one round).
    constexpr int kU = 2;
    const int cpr = D / 8;  // 16-byte chunks per row
    const int total = rows * cpr;
    for (int i0 = threadIdx.x; i0 < total; i0 += 256 * kU) {
      u32x4_t xk[kU], xv[kU];
      int ro[kU], co[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = i0 + 256 * u;
        ro[u] = i / cpr;
        co[u] = (i - ro[u] * cpr) * 8;
        if (i < total) {
          xk[u] = ld16(ksrc + ro[u] * k_t + co[u]);
          xv[u] = ld16(vsrc + ro[u] * v_t + co[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (i0 + 256 * u < total) {
          st16_nt(kdst + ro[u] * kc_s + co[u], xk[u]);
          st16_nt(vdst + ro[u] * vc_s + co[u], xv[u]);
        }
    }
  } else {
    const int total = rows * D;
    for (int i = threadIdx.x; i < total; i += 256) {
      const int r = i / D, d = i - r * D;
      kdst[r * kc_s + d * kc_d] = ksrc[r * k_t + d * k_d];
      vdst[r * vc_s + d * vc_d] = vsrc[r * v_t + d * v_d];
    }
  }
}

// ------------------------------------------------- varlen fill with RoPE --
// The K/V half of the prefill attention block: the varlen fill above, with
// each K row rotated on dims [0, R) at its token's position id before it is
// written, to the page and to the packed roped-K buffer the attention kernel
// reads.  The rotation is the standalone RoPE's device math (rope_sincos,
// rope_rotate, one bf16 rounding), so the pages hold exactly what
// partial_rope followed by paged_kv_fill_varlen writes
// (engine/runner.py:338-340, 381-384).  One workgroup per (logical page, KV
// head, sequence), as the plain fill; the page's sin/cos go to LDS and, from
// the head-0 workgroup, to tab[t] = [sin of the R/2 angles | cos] for the
// attention kernel's q rotation.  Work units: a rotated chunk pair
// (c, c + R/16) of one row, an unrotated K chunk, a V chunk.  Each thread
// requests all of its units' chunks before it computes or stores any
// (kRopeFillUnits per pass), so a pass costs one memory round trip.
constexpr int kRopeFillUnits = 4;
constexpr int kRopeFillMaxR = 128;

__global__ __launch_bounds__(256) void prefill_kv_rope_fill_kernel(
    bf16_t *__restrict__ kc, bf16_t *__restrict__ vc, int64_t kc_p, int64_t kc_h,
    int64_t kc_s, int64_t vc_p, int64_t vc_h, int64_t vc_s, const bf16_t *__restrict__ k,
    int64_t k_t, int64_t k_h, const bf16_t *__restrict__ v, int64_t v_t, int64_t v_h,
    bf16_t *__restrict__ kr, int64_t kr_t, int64_t kr_h, float *__restrict__ tab,
    const int32_t *__restrict__ bt, int64_t bt_b, const int32_t *__restrict__ cu,
    const void *__restrict__ pos, int64_t ps_t, int pos64, const float *__restrict__ inv_freq,
    int R, int D, int H) {
  __shared__ float sn_l[kPage][kRopeFillMaxR / 2], cs_l[kPage][kRopeFillMaxR / 2];
  const int lp = blockIdx.x, h0 = blockIdx.y, b = blockIdx.z;
  const int start = cu[b];
  const int n = cu[b + 1] - start;
  const int t0 = lp * kPage;
  if (t0 >= n) return;
  const int rows = min(kPage, n - t0);
  const int64_t phys = int64_t(bt[b * bt_b + lp]);
  const int64_t tok0 = int64_t(start) + t0;
  const int cpr = D / 8, hr = R / 16;   // chunks per row; rotated chunk pairs per row
  const int kcopy = cpr - 2 * hr;       // unrotated K chunks per (row, head)
  const int n_rot = rows * hr, n_kcopy = rows * kcopy;
  const int total = n_rot + n_kcopy + rows * cpr;
  const int h = h0;
  const int half = R / 2;
  for (int base = 0; base < total; base += 256 * kRopeFillUnits) {
    // 1. request every chunk of this pass
    u32x4_t x0[kRopeFillUnits], x1[kRopeFillUnits];
#pragma unroll
    for (int u = 0; u < kRopeFillUnits; ++u) {
      const int i = base + u * 256 + int(threadIdx.x);
      x0[u] = x1[u] = u32x4_t{0u, 0u, 0u, 0u};
      if (i < n_rot) {
        const int r = i / hr, c = i - r * hr;
        const bf16_t *src = k + h * k_h + (tok0 + r) * k_t + c * 8;
        x0[u] = ld16(src);
        x1[u] = ld16(src + half);
      } else if (i < n_rot + n_kcopy) {
        const int j = i - n_rot;
        const int r = j / kcopy, c = 2 * hr + (j - r * kcopy);
        x0[u] = ld16(k + h * k_h + (tok0 + r) * k_t + c * 8);
      } else if (i < total) {
        const int j = i - n_rot - n_kcopy;
        const int r = j / cpr, c = j - r * cpr;
        x0[u] = ld16(v + h * v_h + (tok0 + r) * v_t + c * 8);
      }
    }
    // 2. the page's sin / cos (first pass only; overlaps the loads)
    if (base == 0) {
      for (int e = threadIdx.x; e < rows * half; e += 256) {
        const int r = e / half, jj = e - r * half;
        float sv, cv;
        rope_sincos(load_pos(pos, (tok0 + r) * ps_t, pos64 != 0), inv_freq[jj], sv, cv);
        sn_l[r][jj] = sv;
        cs_l[r][jj] = cv;
        if (tab && h == 0) {
          tab[(tok0 + r) * R + jj] = sv;
          tab[(tok0 + r) * R + half + jj] = cv;
        }
      }
      __syncthreads();
    }
    // 3. rotate / store
#pragma unroll
    for (int u = 0; u < kRopeFillUnits; ++u) {
      const int i = base + u * 256 + int(threadIdx.x);
      if (i < n_rot) {
        const int r = i / hr, c = i - r * hr;
        u32x4_t oa, ob;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int j0 = c * 8 + 2 * w;
          float o1l, o2l, o1h, o2h;
          rope_rotate(bf16_lo(x0[u][w]), bf16_lo(x1[u][w]), cs_l[r][j0], sn_l[r][j0], o1l, o2l);
          rope_rotate(bf16_hi(x0[u][w]), bf16_hi(x1[u][w]), cs_l[r][j0 + 1], sn_l[r][j0 + 1],
                      o1h, o2h);
          oa[w] = pack_bf16x2(o1l, o1h);
          ob[w] = pack_bf16x2(o2l, o2h);
        }
        bf16_t *dst = kc + phys * kc_p + h * kc_h + r * kc_s + c * 8;
        bf16_t *kdup = kr + h * kr_h + (tok0 + r) * kr_t + c * 8;
        st16_nt(dst, oa);
        st16_nt(dst + half, ob);
        st16_nt(kdup, oa);
        st16_nt(kdup + half, ob);
      } else if (i < n_rot + n_kcopy) {
        const int j = i - n_rot;
        const int r = j / kcopy, c = 2 * hr + (j - r * kcopy);
        st16_nt(kc + phys * kc_p + h * kc_h + r * kc_s + c * 8, x0[u]);
        st16_nt(kr + h * kr_h + (tok0 + r) * kr_t + c * 8, x0[u]);
      } else if (i < total) {
        const int j = i - n_rot - n_kcopy;
        const int r = j / cpr, c = j - r * cpr;
        st16_nt(vc + phys * vc_p + h * vc_h + r * vc_s + c * 8, x0[u]);
      }
    }
  }
}

}  // namespace

extern "C" int wy_prefill_kv_rope_fill(void *k_cache, void *v_cache, const int64_t *kcs,
                                       const int64_t *vcs, const void *k, const int64_t *ks,
                                       const void *v, const int64_t *vs, void *k_roped,
                                       const int64_t *krs, float *rope_table,
                                       const int32_t *block_table,
                                       int64_t bt_stride0, const int32_t *cu_seqlens,
                                       const void *position_ids, int64_t pos_stride,
                                       int pos_is_int64, const float *inv_freq, int rotary_dim,
                                       int batch, int num_kv_heads, int head_dim,
                                       int max_seqlen, void *stream) {
  if (!k_cache || !v_cache || !kcs || !vcs || !k || !ks || !v || !vs || !k_roped || !krs ||
      !block_table || !cu_seqlens || !position_ids || !inv_freq)
    return WY_E_NULL;
  if (batch < 0 || num_kv_heads <= 0 || head_dim <= 0 || max_seqlen < 0) return WY_E_SHAPE;
  if (head_dim % 8 || rotary_dim <= 0 || rotary_dim % 16 || rotary_dim > head_dim ||
      rotary_dim > kRopeFillMaxR)
    return WY_E_SHAPE;
  const bool vec = kcs[3] == 1 && vcs[3] == 1 && ks[2] == 1 && vs[2] == 1 && krs[2] == 1 &&
                   kcs[0] % 8 == 0 && kcs[1] % 8 == 0 && kcs[2] % 8 == 0 && vcs[0] % 8 == 0 &&
                   vcs[1] % 8 == 0 && vcs[2] % 8 == 0 && ks[0] % 8 == 0 && ks[1] % 8 == 0 &&
                   vs[0] % 8 == 0 && vs[1] % 8 == 0 && krs[0] % 8 == 0 && krs[1] % 8 == 0 &&
                   wyh::aligned16(k_cache) && wyh::aligned16(v_cache) && wyh::aligned16(k) &&
                   wyh::aligned16(v) && wyh::aligned16(k_roped);
  if (!vec) return WY_E_LAYOUT;
  if (batch == 0 || max_seqlen == 0) return WY_OK;
  if (rope_table && (reinterpret_cast<uintptr_t>(rope_table) & 15u)) return WY_E_LAYOUT;
  dim3 grid((max_seqlen + kPage - 1) / kPage, num_kv_heads, batch);
  prefill_kv_rope_fill_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<bf16_t *>(k_cache), static_cast<bf16_t *>(v_cache), kcs[0], kcs[1], kcs[2],
      vcs[0], vcs[1], vcs[2], static_cast<const bf16_t *>(k), ks[0], ks[1],
      static_cast<const bf16_t *>(v), vs[0], vs[1], static_cast<bf16_t *>(k_roped), krs[0],
      krs[1], rope_table, block_table, bt_stride0, cu_seqlens, position_ids, pos_stride,
      pos_is_int64, inv_freq, rotary_dim, head_dim, num_kv_heads);
  return wyh::launch_status();
}

extern "C" int wy_paged_kv_append(void *k_cache, void *v_cache, const int64_t *kcs,
                                  const int64_t *vcs, const void *k_new,
                                  const void *v_new, const int64_t *kns,
                                  const int64_t *vns, const int32_t *block_table,
                                  int64_t bt_stride0, const int64_t *pos, int batch,
                                  int num_kv_heads, int head_dim, void *stream) {
  if (!k_cache || !v_cache || !kcs || !vcs || !k_new || !v_new || !kns || !vns ||
      !block_table || !pos)
    return WY_E_NULL;
  if (batch < 0 || num_kv_heads <= 0 || head_dim <= 0) return WY_E_SHAPE;
  if (batch == 0) return WY_OK;
  const bool vec = head_dim % 8 == 0 && kcs[3] == 1 && vcs[3] == 1 && kns[2] == 1 &&
                   vns[2] == 1 && kcs[0] % 8 == 0 && kcs[1] % 8 == 0 &&
                   kcs[2] % 8 == 0 && vcs[0] % 8 == 0 && vcs[1] % 8 == 0 &&
                   vcs[2] % 8 == 0 && kns[0] % 8 == 0 && kns[1] % 8 == 0 &&
                   vns[0] % 8 == 0 && vns[1] % 8 == 0 && wyh::aligned16(k_cache) &&
                   wyh::aligned16(v_cache) && wyh::aligned16(k_new) &&
                   wyh::aligned16(v_new);
  dim3 grid(batch, num_kv_heads);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define WY_APPEND_ARGS                                                            \
  static_cast<bf16_t *>(k_cache), static_cast<bf16_t *>(v_cache), kcs[0], kcs[1], \
      kcs[2], kcs[3], vcs[0], vcs[1], vcs[2], vcs[3],                             \
      static_cast<const bf16_t *>(k_new), static_cast<const bf16_t *>(v_new),     \
      kns[0], kns[1], kns[2], vns[0], vns[1], vns[2], block_table, bt_stride0, pos, \
      head_dim
  if (vec)
    paged_kv_append_kernel<true><<<grid, 64, 0, s>>>(WY_APPEND_ARGS);
  else
    paged_kv_append_kernel<false><<<grid, 64, 0, s>>>(WY_APPEND_ARGS);
#undef WY_APPEND_ARGS
  return wyh::launch_status();
}

extern "C" int wy_paged_kv_fill_varlen(void *k_cache, void *v_cache,
                                       const int64_t *kcs, const int64_t *vcs,
                                       const void *k_packed, const void *v_packed,
                                       const int64_t *ks, const int64_t *vs,
                                       const int32_t *block_table,
                                       int64_t bt_stride0, const int32_t *cu_seqlens,
                                       int batch, int num_kv_heads, int head_dim,
                                       int max_seqlen, void *stream) {
  if (!k_cache || !v_cache || !kcs || !vcs || !k_packed || !v_packed || !ks || !vs ||
      !block_table || !cu_seqlens)
    return WY_E_NULL;
  if (batch < 0 || num_kv_heads <= 0 || head_dim <= 0 || max_seqlen < 0)
    return WY_E_SHAPE;
  if (batch == 0 || max_seqlen == 0) return WY_OK;
  const bool vec = head_dim % 8 == 0 && kcs[3] == 1 && vcs[3] == 1 && ks[2] == 1 &&
                   vs[2] == 1 && kcs[0] % 8 == 0 && kcs[1] % 8 == 0 &&
                   kcs[2] % 8 == 0 && vcs[0] % 8 == 0 && vcs[1] % 8 == 0 &&
                   vcs[2] % 8 == 0 && ks[0] % 8 == 0 && ks[1] % 8 == 0 &&
                   vs[0] % 8 == 0 && vs[1] % 8 == 0 && wyh::aligned16(k_cache) &&
                   wyh::aligned16(v_cache) && wyh::aligned16(k_packed) &&
                   wyh::aligned16(v_packed);
  dim3 grid((max_seqlen + kPage - 1) / kPage, num_kv_heads, batch);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define WY_FILL_ARGS                                                              \
  static_cast<bf16_t *>(k_cache), static_cast<bf16_t *>(v_cache), kcs[0], kcs[1], \
      kcs[2], kcs[3], vcs[0], vcs[1], vcs[2], vcs[3],                             \
      static_cast<const bf16_t *>(k_packed), static_cast<const bf16_t *>(v_packed), \
      ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], block_table, bt_stride0,          \
      cu_seqlens, head_dim
  if (vec)
    paged_kv_fill_varlen_kernel<true><<<grid, 256, 0, s>>>(WY_FILL_ARGS);
  else
    paged_kv_fill_varlen_kernel<false><<<grid, 256, 0, s>>>(WY_FILL_ARGS);
#undef WY_FILL_ARGS
  return wyh::launch_status();
}
