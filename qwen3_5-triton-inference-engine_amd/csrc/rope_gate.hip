// Elementwise members of the path: partial rotate-half RoPE and the sigmoid
// output-gate pack.  Both are HBM streams; the fast paths move 16-byte chunks
// (8 bf16) per lane, the generic paths one element per lane for layouts with a
// non-unit innermost stride.
#include "wy_common.h"

using namespace wy;

namespace {

__device__ __forceinline__ float load_pos(const void *pos, int64_t off, bool is64) {
  return is64 ? float(static_cast<const int64_t *>(pos)[off])
              : float(static_cast<const int32_t *>(pos)[off]);
}

// ------------------------------------------------------------ partial RoPE --
// Fast path: lanes own 16-byte chunks of a row.  A chunk in the first rotary
// half also produces its partner chunk R/2 further on; chunks of the second
// half idle; tail chunks are copied verbatim.  Reference: partial_rope.py:34-132.
__global__ __launch_bounds__(256) void partial_rope_vec_kernel(
    const bf16_t *__restrict__ x, int64_t xs_b, int64_t xs_h, int64_t xs_t,
    bf16_t *__restrict__ out, int64_t os_b, int64_t os_h, int64_t os_t,
    const void *__restrict__ pos, int64_t ps_b, int64_t ps_t, int pos64,
    const float *__restrict__ inv_freq, int H, int T, int D, int R, int64_t rows) {
  const int cpr = D / 8;
  const int64_t gid = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = gid / cpr;
  if (row >= rows) return;
  const int c = int(gid - row * cpr);
  const int t = int(row % T);
  const int64_t bh = row / T;
  const int h = int(bh % H);
  const int b = int(bh / H);
  const bf16_t *xr = x + b * xs_b + h * xs_h + t * xs_t;
  bf16_t *orow = out + b * os_b + h * os_h + t * os_t;
  const int half_chunks = R / 16;
  if (c < half_chunks) {
    const float p = load_pos(pos, b * ps_b + int64_t(t) * ps_t, pos64 != 0);
    const u32x4_t a = ld16(xr + c * 8);
    const u32x4_t bb = ld16(xr + R / 2 + c * 8);
    u32x4_t oa, ob;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float o1l, o2l, o1h, o2h, sl, cl, sh, ch;
      rope_sincos(p, inv_freq[c * 8 + 2 * w], sl, cl);
      rope_sincos(p, inv_freq[c * 8 + 2 * w + 1], sh, ch);
      rope_rotate(bf16_lo(a[w]), bf16_lo(bb[w]), cl, sl, o1l, o2l);
      rope_rotate(bf16_hi(a[w]), bf16_hi(bb[w]), ch, sh, o1h, o2h);
      oa[w] = pack_bf16x2(o1l, o1h);
      ob[w] = pack_bf16x2(o2l, o2h);
    }
    st16(orow + c * 8, oa);
    st16(orow + R / 2 + c * 8, ob);
  } else if (c >= 2 * half_chunks) {
    st16(orow + c * 8, ld16(xr + c * 8));
  }
}

// Generic path: one lane per output element, any strides, any even R <= D.
__global__ __launch_bounds__(256) void partial_rope_generic_kernel(
    const bf16_t *__restrict__ x, int64_t xs_b, int64_t xs_h, int64_t xs_t,
    int64_t xs_d, bf16_t *__restrict__ out, int64_t os_b, int64_t os_h, int64_t os_t,
    int64_t os_d, const void *__restrict__ pos, int64_t ps_b, int64_t ps_t, int pos64,
    const float *__restrict__ inv_freq, int H, int T, int D, int R, int64_t total) {
  const int64_t gid = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= total) return;
  const int d = int(gid % D);
  const int64_t row = gid / D;
  const int t = int(row % T);
  const int64_t bh = row / T;
  const int h = int(bh % H);
  const int b = int(bh / H);
  const bf16_t *xr = x + b * xs_b + h * xs_h + t * xs_t;
  bf16_t *o = out + b * os_b + h * os_h + t * os_t + d * os_d;
  const int half = R / 2;
  if (d >= R) {
    *o = xr[d * xs_d];
    return;
  }
  const int j = d < half ? d : d - half;
  const float p = load_pos(pos, b * ps_b + int64_t(t) * ps_t, pos64 != 0);
  float s, c;
  rope_sincos(p, inv_freq[j], s, c);
  const float x1 = bf16_to_f32(xr[j * xs_d]);
  const float x2 = bf16_to_f32(xr[(j + half) * xs_d]);
  float o1, o2;
  rope_rotate(x1, x2, c, s, o1, o2);
  *o = bf16_t(f32_to_bf16_bits(d < half ? o1 : o2));
}

// ------------------------------------------------------- gate pack (fast) --
// Lanes own 16-byte chunks of the packed output row [t, h*D + 8c .. +8).
// Reference: attention_gate_pack.py:20-63.
__global__ __launch_bounds__(256) void gate_pack_vec_kernel(
    const bf16_t *__restrict__ x, int64_t xs_h, int64_t xs_t,
    const bf16_t *__restrict__ g, int64_t gs_h, int64_t gs_t, bf16_t *__restrict__ out,
    int H, int D, int64_t chunks) {
  const int64_t gid = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= chunks) return;
  const int cpt = H * D / 8;  // chunks per token
  const int64_t t = gid / cpt;
  const int r = int(gid - t * cpt);
  const int h = r / (D / 8), c = (r - h * (D / 8)) * 8;
  const u32x4_t xv = ld16(x + h * xs_h + t * xs_t + c);
  const u32x4_t gv = ld16(g + h * gs_h + t * gs_t + c);
  u32x4_t o;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float sl = 1.0f / (1.0f + __expf(-bf16_lo(gv[w])));
    const float sh = 1.0f / (1.0f + __expf(-bf16_hi(gv[w])));
    o[w] = pack_bf16x2(bf16_lo(xv[w]) * sl, bf16_hi(xv[w]) * sh);
  }
  st16(out + gid * 8, o);
}

__global__ __launch_bounds__(256) void gate_pack_generic_kernel(
    const bf16_t *__restrict__ x, int64_t xs_h, int64_t xs_t, int64_t xs_d,
    const bf16_t *__restrict__ g, int64_t gs_h, int64_t gs_t, int64_t gs_d,
    bf16_t *__restrict__ out, int H, int D, int64_t total) {
  const int64_t gid = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= total) return;
  const int64_t t = gid / (int64_t(H) * D);
  const int r = int(gid - t * H * D);
  const int h = r / D, d = r - h * D;
  const float xv = bf16_to_f32(x[h * xs_h + t * xs_t + d * xs_d]);
  const float gv = bf16_to_f32(g[h * gs_h + t * gs_t + d * gs_d]);
  out[gid] = bf16_t(f32_to_bf16_bits(xv * (1.0f / (1.0f + __expf(-gv)))));
}

inline unsigned blocks_for(int64_t n) { return unsigned((n + 255) / 256); }

}  // namespace

extern "C" int wy_partial_rope(const void *x, const int64_t *xs, void *out,
                               const int64_t *os, const void *position_ids,
                               const int64_t *ps, int pos_is_int64,
                               const float *inv_freq, int batch, int num_heads,
                               int num_tokens, int head_dim, int rotary_dim,
                               void *stream) {
  if (!x || !xs || !out || !os || !position_ids || !ps || !inv_freq) return WY_E_NULL;
  if (batch < 0 || num_heads < 0 || num_tokens < 0 || head_dim <= 0 ||
      rotary_dim <= 0 || rotary_dim > head_dim || rotary_dim % 2 != 0)
    return WY_E_SHAPE;
  const int64_t rows = int64_t(batch) * num_heads * num_tokens;
  if (rows == 0) return WY_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = head_dim % 8 == 0 && rotary_dim % 16 == 0 && xs[3] == 1 &&
                   os[3] == 1 && xs[0] % 8 == 0 && xs[1] % 8 == 0 && xs[2] % 8 == 0 &&
                   os[0] % 8 == 0 && os[1] % 8 == 0 && os[2] % 8 == 0 &&
                   wyh::aligned16(x) && wyh::aligned16(out);
  if (vec) {
    const int64_t n = rows * (head_dim / 8);
    partial_rope_vec_kernel<<<blocks_for(n), 256, 0, s>>>(
        static_cast<const bf16_t *>(x), xs[0], xs[1], xs[2], static_cast<bf16_t *>(out),
        os[0], os[1], os[2], position_ids, ps[0], ps[1], pos_is_int64, inv_freq,
        num_heads, num_tokens, head_dim, rotary_dim, rows);
  } else {
    const int64_t n = rows * head_dim;
    partial_rope_generic_kernel<<<blocks_for(n), 256, 0, s>>>(
        static_cast<const bf16_t *>(x), xs[0], xs[1], xs[2], xs[3],
        static_cast<bf16_t *>(out), os[0], os[1], os[2], os[3], position_ids, ps[0],
        ps[1], pos_is_int64, inv_freq, num_heads, num_tokens, head_dim, rotary_dim, n);
  }
  return wyh::launch_status();
}

extern "C" int wy_attention_gate_pack(const void *x, const int64_t *xs, const void *gate,
                                      const int64_t *gs, void *out, int num_heads,
                                      int num_tokens, int head_dim, void *stream) {
  if (!x || !xs || !gate || !gs || !out) return WY_E_NULL;
  if (num_heads < 0 || num_tokens < 0 || head_dim <= 0) return WY_E_SHAPE;
  const int64_t total = int64_t(num_tokens) * num_heads * head_dim;
  if (total == 0) return WY_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // x/gate strides are [b, h, t, d]; batch is 1 so the b stride is unused.
  const bool vec = head_dim % 8 == 0 && xs[3] == 1 && gs[3] == 1 && xs[1] % 8 == 0 &&
                   xs[2] % 8 == 0 && gs[1] % 8 == 0 && gs[2] % 8 == 0 &&
                   wyh::aligned16(x) && wyh::aligned16(gate) && wyh::aligned16(out);
  if (vec) {
    const int64_t chunks = total / 8;
    gate_pack_vec_kernel<<<blocks_for(chunks), 256, 0, s>>>(
        static_cast<const bf16_t *>(x), xs[1], xs[2], static_cast<const bf16_t *>(gate),
        gs[1], gs[2], static_cast<bf16_t *>(out), num_heads, head_dim, chunks);
  } else {
    gate_pack_generic_kernel<<<blocks_for(total), 256, 0, s>>>(
        static_cast<const bf16_t *>(x), xs[1], xs[2], xs[3],
        static_cast<const bf16_t *>(gate), gs[1], gs[2], gs[3],
        static_cast<bf16_t *>(out), num_heads, head_dim, total);
  }
  return wyh::launch_status();
}
