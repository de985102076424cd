// Elementwise members of the path: partial rotate-half RoPE and the sigmoid
// output-gate pack.  Both are HBM streams; the fast paths move 16-byte chunks
// (8 bf16) per lane, the generic paths one element per lane for layouts with a
// non-unit innermost stride.
#include "wy_common.h"

using namespace wy;

namespace {


// ------------------------------------------------------------ partial RoPE --
// Fast path.  The grid's first part rotates: a lane owns dims 2c, 2c + 1 of
// the first rotary half of one (b, t) row for two heads, so its 2 sin/cos
// pairs (which depend on (b, t, j) only) serve both; each head's pair and
// partner pair (dims + R/2) are rotated together.  (Two dims per lane rather
// than a 16-byte chunk of eight: the accurate sin/cos cost tens of VALU
// instructions each, and eight in a row made the rotating lanes the launch's
// critical path when there are few heads.)
// The second part copies the tail chunks [R/8, D/8) of every (b, t, h) row.
// The two kinds of work sit in different wavefronts, so neither waits on the
// other's branch.  Reference: partial_rope.py:34-132.
constexpr int kRopeHeads = 2;  // heads per rotating lane
constexpr int kRopeDims = 2;   // first-half dims per rotating lane

__global__ __launch_bounds__(256) void partial_rope_vec_kernel(
    const bf16_t *__restrict__ x, int64_t xs_b, int64_t xs_h, int64_t xs_t,
    bf16_t *__restrict__ out, int64_t os_b, int64_t os_h, int64_t os_t,
    const void *__restrict__ pos, int64_t ps_b, int64_t ps_t, int pos64,
    const float *__restrict__ inv_freq, int H, int T, int D, int R, uint32_t bt_rows) {
  // index math in 32 bits: the host launches this kernel only when the grid
  // and row counts fit
  const uint32_t half_units = uint32_t(R) / (2u * kRopeDims);
  const uint32_t hgroups = uint32_t(H + kRopeHeads - 1) / kRopeHeads;
  const uint32_t n_rot = bt_rows * half_units * hgroups;
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  if (gid < n_rot) {
    // lane -> (b, t, head group, unit), unit fastest
    const uint32_t q1 = gid / half_units;
    const int c = int(gid - q1 * half_units);
    const uint32_t bt = q1 / hgroups;
    const int h0 = int(q1 - bt * hgroups) * kRopeHeads;
    const int t = int(bt % uint32_t(T)), b = int(bt / uint32_t(T));
    const bf16_t *xr = x + b * xs_b + t * xs_t;
    bf16_t *orow = out + b * os_b + t * os_t;
    const float p = load_pos(pos, b * ps_b + int64_t(t) * ps_t, pos64 != 0);
    uint32_t a[kRopeHeads], bb[kRopeHeads];
#pragma unroll
    for (int i = 0; i < kRopeHeads; ++i) {
      const int h = min(h0 + i, H - 1);
      a[i] = *reinterpret_cast<const uint32_t *>(xr + h * xs_h + c * kRopeDims);
      bb[i] = *reinterpret_cast<const uint32_t *>(xr + h * xs_h + R / 2 + c * kRopeDims);
    }
    float sn[kRopeDims], cs[kRopeDims];
#pragma unroll
    for (int e = 0; e < kRopeDims; ++e)
      rope_sincos(p, inv_freq[c * kRopeDims + e], sn[e], cs[e]);
#pragma unroll
    for (int i = 0; i < kRopeHeads; ++i) {
      if (h0 + i >= H) break;
      float o1l, o2l, o1h, o2h;
      rope_rotate(bf16_lo(a[i]), bf16_lo(bb[i]), cs[0], sn[0], o1l, o2l);
      rope_rotate(bf16_hi(a[i]), bf16_hi(bb[i]), cs[1], sn[1], o1h, o2h);
      __builtin_nontemporal_store(pack_bf16x2(o1l, o1h),
                                  reinterpret_cast<uint32_t *>(orow + (h0 + i) * os_h + c * kRopeDims));
      __builtin_nontemporal_store(
          pack_bf16x2(o2l, o2h),
          reinterpret_cast<uint32_t *>(orow + (h0 + i) * os_h + R / 2 + c * kRopeDims));
    }
    return;
  }
  // rows in memory order: heads fastest when x's head stride is the smaller
  // one (the [T, H, D] buffer the prefill passes as a permuted view), tokens
  // fastest otherwise
  const uint32_t tail = uint32_t(D - R) / 8u;
  if (tail == 0) return;  // R == D: no tail (and no division by zero)
  const uint32_t k = gid - n_rot;
  const uint32_t row = k / tail;
  if (row >= bt_rows * uint32_t(H)) return;
  const int c = R / 8 + int(k - row * tail);
  int t, h, b;
  if (xs_h < xs_t) {
    h = int(row % uint32_t(H));
    const uint32_t bt = row / uint32_t(H);
    t = int(bt % uint32_t(T));
    b = int(bt / uint32_t(T));
  } else {
    t = int(row % uint32_t(T));
    const uint32_t bh = row / uint32_t(T);
    h = int(bh % uint32_t(H));
    b = int(bh / uint32_t(H));
  }
  st16_nt(out + b * os_b + h * os_h + t * os_t + c * 8, ld16(x + b * xs_b + h * xs_h + t * xs_t + c * 8));
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
    const float sl = gate_sigmoid(bf16_lo(gv[w]));
    const float sh = gate_sigmoid(bf16_hi(gv[w]));
    o[w] = pack_bf16x2(bf16_lo(xv[w]) * sl, bf16_hi(xv[w]) * sh);
  }
  st16_nt(out + gid * 8, o);
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
  out[gid] = bf16_t(f32_to_bf16_bits(xv * gate_sigmoid(gv)));
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
  // fast path: rotating lanes (2 dims x 2 heads each) + tail lanes (one
  // 16-byte chunk each), counted in 32 bits
  const int64_t bt_rows = int64_t(batch) * num_tokens;
  const int64_t n_vec = bt_rows * (rotary_dim / 4) * ((num_heads + 1) / 2) +
                        bt_rows * num_heads * (head_dim / 8 - rotary_dim / 8);
  const bool vec = head_dim % 8 == 0 && rotary_dim % 16 == 0 && xs[3] == 1 &&
                   n_vec + 256 < int64_t(INT32_MAX) &&
                   os[3] == 1 && xs[0] % 8 == 0 && xs[1] % 8 == 0 && xs[2] % 8 == 0 &&
                   os[0] % 8 == 0 && os[1] % 8 == 0 && os[2] % 8 == 0 &&
                   wyh::aligned16(x) && wyh::aligned16(out);
  if (vec) {
    partial_rope_vec_kernel<<<blocks_for(n_vec), 256, 0, s>>>(
        static_cast<const bf16_t *>(x), xs[0], xs[1], xs[2], static_cast<bf16_t *>(out),
        os[0], os[1], os[2], position_ids, ps[0], ps[1], pos_is_int64, inv_freq,
        num_heads, num_tokens, head_dim, rotary_dim, uint32_t(bt_rows));
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
