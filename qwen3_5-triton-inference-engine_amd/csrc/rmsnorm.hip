// Per-row RMSNorm with a (1 + w) weight (Qwen's q/k head norm), bf16 in/out,
// fp32 math.  A row is owned by 32 consecutive lanes; lane l holds elements
// 8(32k + l) .. +7 of each 256-element block k.  The reduction order is the
// one rms_rsigma() fixes, shared with the fused decode attention block.
// Reference: qwen_rmsnorm.py:28-90 (kernel), :92-147 (op).
#include "wy_common.h"

using namespace wy;

namespace {

constexpr int kRowsPerBlock = 8;  // 256 threads

__global__ __launch_bounds__(256) void qwen_rmsnorm_kernel(
    const bf16_t *__restrict__ x, int64_t xs_b, int64_t xs_m, const bf16_t *__restrict__ w,
    bf16_t *__restrict__ out, int64_t os_b, int64_t os_m, int rows, int D, float eps) {
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 5);
  if (row >= rows) return;  // uniform over the row's 32 lanes
  const int l = threadIdx.x & 31;
  const bf16_t *xr = x + blockIdx.y * xs_b + row * xs_m;
  bf16_t *orow = out + blockIdx.y * os_b + row * os_m;
  const int nk = D / 256;
  float ss = 0.f;
  for (int k = 0; k < nk; ++k) {
    ss = rms_acc8(ld16(xr + (32 * k + l) * 8), ss);
  }
  const float rs = rms_rsigma(ss, D, eps);
  for (int k = 0; k < nk; ++k) {
    const int c = (32 * k + l) * 8;
    const u32x4_t xw = ld16(xr + c);
    const u32x4_t ww = ld16(w + c);
    u32x4_t y;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      y[e] = pack_bf16x2(rms_apply(bf16_lo(xw[e]), rs, bf16_lo(ww[e])),
                         rms_apply(bf16_hi(xw[e]), rs, bf16_hi(ww[e])));
    st16(orow + c, y);
  }
}

// Residual add fused with the RMSNorm that follows it in a decoder layer:
// sum = bf16(h + x) (the residual add, rounded as a separate add would round
// it), normed = RMSNorm(sum).  The sum of squares runs over the rounded sum in
// qwen_rmsnorm_kernel's order, so both outputs equal the two separate ops bit
// for bit.  Rows contiguous, [rows, kNK * 256]; a lane's kNK chunks of h, x
// and w are all requested before the first is used (one memory round trip
// per row: the op sits on the decode step's serial chain).
template <int kNK>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(
    const bf16_t *__restrict__ h, const bf16_t *__restrict__ x, const bf16_t *__restrict__ w,
    bf16_t *__restrict__ sum, bf16_t *__restrict__ out, int rows, float eps) {
  constexpr int D = kNK * 256;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 5);
  if (row >= rows) return;  // uniform over the row's 32 lanes
  const int l = threadIdx.x & 31;
  const int64_t base = int64_t(row) * D;
  u32x4_t a[kNK], b[kNK], ww[kNK];
#pragma unroll
  for (int k = 0; k < kNK; ++k) {
    const int c = (32 * k + l) * 8;
    a[k] = ld16(h + base + c);
    b[k] = ld16(x + base + c);
    ww[k] = ld16(w + c);
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNK; ++k) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      a[k][e] = pack_bf16x2(bf16_lo(a[k][e]) + bf16_lo(b[k][e]),
                            bf16_hi(a[k][e]) + bf16_hi(b[k][e]));
    st16(sum + base + (32 * k + l) * 8, a[k]);
    ss = rms_acc8(a[k], ss);
  }
  const float rs = rms_rsigma(ss, D, eps);
#pragma unroll
  for (int k = 0; k < kNK; ++k) {
    u32x4_t y;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      y[e] = pack_bf16x2(rms_apply(bf16_lo(a[k][e]), rs, bf16_lo(ww[k][e])),
                         rms_apply(bf16_hi(a[k][e]), rs, bf16_hi(ww[k][e])));
    st16(out + base + (32 * k + l) * 8, y);
  }
}

}  // namespace

extern "C" int wy_qwen_rmsnorm(const void *x, const int64_t *xs, const void *weight, void *out,
                               const int64_t *os, int batch, int rows, int d_model, float eps,
                               void *stream) {
  if (!x || !xs || !weight || !out || !os) return WY_E_NULL;
  if (batch < 0 || rows < 0 || d_model <= 0) return WY_E_SHAPE;
  if (d_model % 256 != 0) return WY_E_UNSUPPORTED;
  if (xs[2] != 1 || os[2] != 1 || xs[0] % 8 || xs[1] % 8 || os[0] % 8 || os[1] % 8 ||
      !wyh::aligned16(x) || !wyh::aligned16(weight) || !wyh::aligned16(out))
    return WY_E_LAYOUT;
  if (batch == 0 || rows == 0) return WY_OK;
  const dim3 grid(unsigned((rows + kRowsPerBlock - 1) / kRowsPerBlock), unsigned(batch));
  qwen_rmsnorm_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(x), xs[0], xs[1], static_cast<const bf16_t *>(weight),
      static_cast<bf16_t *>(out), os[0], os[1], rows, d_model, eps);
  return wyh::launch_status();
}

extern "C" int wy_add_rmsnorm(const void *h, const void *x, const void *weight, void *sum,
                              void *out, int rows, int d_model, float eps, void *stream) {
  if (!h || !x || !weight || !sum || !out) return WY_E_NULL;
  if (rows < 0 || d_model <= 0) return WY_E_SHAPE;
  if (d_model % 256 != 0 || d_model > 1024) return WY_E_UNSUPPORTED;
  if (!wyh::aligned16(h) || !wyh::aligned16(x) || !wyh::aligned16(weight) ||
      !wyh::aligned16(sum) || !wyh::aligned16(out))
    return WY_E_LAYOUT;
  if (rows == 0) return WY_OK;
  const dim3 grid(unsigned((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  const auto *hb = static_cast<const bf16_t *>(h), *xb = static_cast<const bf16_t *>(x);
  const auto *wb = static_cast<const bf16_t *>(weight);
  auto *sb = static_cast<bf16_t *>(sum), *ob = static_cast<bf16_t *>(out);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (d_model / 256) {
    case 1: add_rmsnorm_kernel<1><<<grid, 256, 0, st>>>(hb, xb, wb, sb, ob, rows, eps); break;
    case 2: add_rmsnorm_kernel<2><<<grid, 256, 0, st>>>(hb, xb, wb, sb, ob, rows, eps); break;
    case 3: add_rmsnorm_kernel<3><<<grid, 256, 0, st>>>(hb, xb, wb, sb, ob, rows, eps); break;
    case 4: add_rmsnorm_kernel<4><<<grid, 256, 0, st>>>(hb, xb, wb, sb, ob, rows, eps); break;
    default: return WY_E_UNSUPPORTED;
  }
  return wyh::launch_status();
}
