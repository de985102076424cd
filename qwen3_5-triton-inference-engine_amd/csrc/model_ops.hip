// The model-level ops of a decode step around the two mixers, on gfx950:
// token embedding gather, residual add, SwiGLU, and the LM head fused with
// the vocabulary argmax (logits never written).
// Reference: embedding_gather.py:20-104, residual_add.py:8-52, swiglu.py:22-111,
// vocab_argmax.py:29-224.
#include "wy_common.h"

using namespace wy;

namespace {

// ---- embedding gather: one 16-byte chunk per thread ------------------------------
__global__ __launch_bounds__(256) void embedding_gather_kernel(
    const void *__restrict__ ids, int ids_is_64, const bf16_t *__restrict__ table,
    int64_t tbl_row, int64_t vocab, bf16_t *__restrict__ out, int64_t out_row, int T,
    int chunks_per_row) {
  const int64_t gid = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int t = int(gid / chunks_per_row);
  const int c = int(gid - int64_t(t) * chunks_per_row);
  if (t >= T) return;
  const int64_t id = ids_is_64 ? static_cast<const int64_t *>(ids)[t]
                               : int64_t(static_cast<const int32_t *>(ids)[t]);
  // an id outside [0, vocab) yields a zero row instead of a read past the table
  const bool ok = id >= 0 && id < vocab;
  st16(out + t * out_row + c * 8,
       ok ? ld16(table + id * tbl_row + c * 8) : u32x4_t{0u, 0u, 0u, 0u});
}

// ---- residual add: bf16(x + r), 8 elements per thread ---------------------------
__global__ __launch_bounds__(256) void residual_add_kernel(const bf16_t *__restrict__ x,
                                                           const bf16_t *__restrict__ r,
                                                           bf16_t *__restrict__ out, int64_t n) {
  const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (i + 8 <= n) {
    const u32x4_t a = ld16(x + i), b = ld16(r + i);
    u32x4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack_bf16x2(bf16_lo(a[e]) + bf16_lo(b[e]), bf16_hi(a[e]) + bf16_hi(b[e]));
    st16(out + i, o);
  } else {
    for (int64_t j = i; j < n; ++j)
      out[j] = bf16_t(f32_to_bf16_bits(bf16_to_f32(x[j]) + bf16_to_f32(r[j])));
  }
}

// ---- SwiGLU: bf16((up * gate) * sigmoid(gate)) -------------------------------------
__device__ __forceinline__ float swiglu1(float g, float u) {
  return (u * g) * (1.0f / (1.0f + __expf(-g)));
}
__global__ __launch_bounds__(256) void swiglu_kernel(const bf16_t *__restrict__ gate,
                                                     int64_t g_m, int64_t g_n,
                                                     const bf16_t *__restrict__ up, int64_t u_m,
                                                     int64_t u_n, bf16_t *__restrict__ out,
                                                     int M, int N, int vec) {
  const int64_t gid = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (vec) {  // unit inner strides, 8 | N, 16-byte aligned rows
    const int cpr = N / 8;
    const int m = int(gid / cpr), c = int(gid - int64_t(m) * cpr) * 8;
    if (m >= M) return;
    const u32x4_t gw = ld16(gate + m * g_m + c), uw = ld16(up + m * u_m + c);
    u32x4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack_bf16x2(swiglu1(bf16_lo(gw[e]), bf16_lo(uw[e])),
                         swiglu1(bf16_hi(gw[e]), bf16_hi(uw[e])));
    st16(out + int64_t(m) * N + c, o);
  } else {
    const int m = int(gid / N), n = int(gid - int64_t(m) * N);
    if (m >= M) return;
    out[int64_t(m) * N + n] = bf16_t(f32_to_bf16_bits(
        swiglu1(bf16_to_f32(gate[m * g_m + n * g_n]), bf16_to_f32(up[m * u_m + n * u_n]))));
  }
}

// ---- LM head + argmax -----------------------------------------------------------------
//
// logits[m, v] = sum_k x[m, k] W[v, k] (fp32), token[m] = argmax_v (first
// index on ties).  Stage 1: persistent 8-wave workgroups stage x (rows
// padded to MT*16, zero rows past the batch) in LDS once, then stream
// 16-row vocabulary tiles straight from HBM into the B operand of
// v_mfma_f32_16x16x32_bf16 (lane = vocab row l%16 x 8 consecutive k), x
// from LDS as the A operand.  Lane l's outputs are rows 4(l/16)+j of column
// l%16; each lane keeps its running best over the tiles it sees (strict
// greater: the first maximum).  The workgroup folds its 8 waves x 16
// columns into one key per row: orderable float bits << 32 | ~index, so the
// largest key is the largest logit with the smallest index.  Stage 2: one
// wavefront per row takes the max key over the workgroups.  NaN ranks above
// every number (first NaN wins), as torch.argmax does, and a lane takes the
// first valid column it sees unconditionally, so a row whose logits are all
// -inf or NaN still yields an index in [0, V).
constexpr int kArgmaxWaves = 8;
constexpr int kKBatch = 8;  // k-steps (32 wide) whose weight loads are in flight together

__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  uint32_t u = __float_as_uint(v);
  u = (v != v) ? 0xffffffffu : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
  return (uint64_t(u) << 32) | uint64_t(0xffffffffu - uint32_t(idx));
}
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  const uint32_t lo = __shfl_xor(uint32_t(v), o), hi = __shfl_xor(uint32_t(v >> 32), o);
  return (uint64_t(hi) << 32) | lo;
}

template <int MT>
__global__ __launch_bounds__(64 * kArgmaxWaves) void lm_head_argmax_stage1(
    const bf16_t *__restrict__ x, int64_t x_row, const bf16_t *__restrict__ w, int64_t w_row,
    uint64_t *__restrict__ partial, int rows, int K, int V) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16_t *xs = reinterpret_cast<bf16_t *>(lds_raw);  // [MT*16][K + 8]
  uint64_t *red = reinterpret_cast<uint64_t *>(lds_raw + size_t(MT) * 16 * (K + 8) * 2);
  const int ldx = K + 8;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // stage x: 16-byte chunks, zero rows past the batch
  const int cpr = K / 8;
  for (int i = threadIdx.x; i < MT * 16 * cpr; i += 64 * kArgmaxWaves) {
    const int m = i / cpr, c = (i - m * cpr) * 8;
    const u32x4_t v = m < rows ? ld16(x + m * x_row + c) : u32x4_t{0u, 0u, 0u, 0u};
    st16(xs + m * ldx + c, v);
  }
  __syncthreads();

  const int n16 = lane & 15, g4 = lane >> 4;
  float best[MT][4];
  int best_i[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      best[mt][j] = -INFINITY;
      best_i[mt][j] = 0x7fffffff;
    }
  const int ntiles = (V + 15) / 16;
  const int stride = gridDim.x * kArgmaxWaves;
  const int ksteps = K / 32;
  for (int tile = blockIdx.x * kArgmaxWaves + wave; tile < ntiles; tile += stride) {
    const int vrow = tile * 16 + n16;
    const bf16_t *wr = w + int64_t(vrow < V ? vrow : V - 1) * w_row + g4 * 8;
    f32x4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < ksteps; k0 += kKBatch) {
      u32x4_t wv[kKBatch];
#pragma unroll
      for (int s = 0; s < kKBatch; ++s) wv[s] = ld16(wr + (k0 + s) * 32);
#pragma unroll
      for (int s = 0; s < kKBatch; ++s) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const u32x4_t xv = ld16(xs + (mt * 16 + n16) * ldx + (k0 + s) * 32 + g4 * 8);
          acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xv),
                                                            __builtin_bit_cast(bf16x8_t, wv[s]),
                                                            acc[mt], 0, 0, 0);
        }
      }
    }
    if (vrow < V) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (best_i[mt][j] == 0x7fffffff || acc[mt][j] > best[mt][j] ||
              (acc[mt][j] != acc[mt][j] && best[mt][j] == best[mt][j])) {
            best[mt][j] = acc[mt][j];
            best_i[mt][j] = vrow;
          }
    }
  }
  // fold: 16 columns of each row group (xor over lane bits 0..3), then waves
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint64_t key = best_i[mt][j] == 0x7fffffff ? 0ull : argmax_key(best[mt][j], best_i[mt][j]);
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) key = max_u64(key, shfl_xor_u64(key, o));
      if (n16 == 0) red[wave * MT * 16 + mt * 16 + g4 * 4 + j] = key;
    }
  __syncthreads();
  for (int m = threadIdx.x; m < MT * 16; m += 64 * kArgmaxWaves) {
    uint64_t key = red[m];
#pragma unroll
    for (int wv = 1; wv < kArgmaxWaves; ++wv) key = max_u64(key, red[wv * MT * 16 + m]);
    if (m < rows) partial[int64_t(m) * gridDim.x + blockIdx.x] = key;
  }
}

__global__ __launch_bounds__(64) void lm_head_argmax_stage2(const uint64_t *__restrict__ partial,
                                                            int nparts, int64_t *__restrict__ out) {
  const int m = blockIdx.x;
  uint64_t key = 0;
  for (int i = threadIdx.x; i < nparts; i += 64) key = max_u64(key, partial[int64_t(m) * nparts + i]);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) key = max_u64(key, shfl_xor_u64(key, o));
  if (threadIdx.x == 0) out[m] = int64_t(0xffffffffu - uint32_t(key & 0xffffffffu));
}

size_t argmax_lds(int rows, int K) {
  const int mt = (rows + 15) / 16;
  return size_t(mt) * 16 * (K + 8) * 2 + size_t(kArgmaxWaves) * mt * 16 * 8;
}
// One round of persistent workgroups: as many per CU as the staged x allows
// (at most 4), 256 CUs on MI355X, never more than there are tile groups.
int argmax_grid(int rows, int K, int V) {
  const int ntiles = (V + 15) / 16;
  const int wgs = (ntiles + kArgmaxWaves - 1) / kArgmaxWaves;
  int per_cu = int((160 * 1024) / argmax_lds(rows, K));
  per_cu = per_cu < 1 ? 1 : (per_cu > 4 ? 4 : per_cu);
  return wgs < 256 * per_cu ? wgs : 256 * per_cu;
}

template <int MT>
int launch_stage1(int grid, size_t lds, hipStream_t st, const bf16_t *x, int64_t xr,
                  const bf16_t *w, int64_t wr, uint64_t *part, int rows, int K, int V) {
  auto *fn = lm_head_argmax_stage1<MT>;
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(fn),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return int(e);
  }
  fn<<<grid, 64 * kArgmaxWaves, lds, st>>>(x, xr, w, wr, part, rows, K, V);
  return wyh::launch_status();
}

}  // namespace

extern "C" int wy_embedding_gather(const void *input_ids, int ids_is_int64, const void *weight,
                                   int64_t weight_row_stride, int64_t vocab, void *out,
                                   int64_t out_row_stride, int tokens, int d_model,
                                   void *stream) {
  if (!input_ids || !weight || !out) return WY_E_NULL;
  if (tokens < 0 || d_model <= 0 || vocab <= 0) return WY_E_SHAPE;
  if (d_model % 8 || weight_row_stride % 8 || out_row_stride % 8 || !wyh::aligned16(weight) ||
      !wyh::aligned16(out))
    return WY_E_LAYOUT;
  if (tokens == 0) return WY_OK;
  const int cpr = d_model / 8;
  const int64_t threads = int64_t(tokens) * cpr;
  embedding_gather_kernel<<<unsigned((threads + 255) / 256), 256, 0,
                            static_cast<hipStream_t>(stream)>>>(
      input_ids, ids_is_int64, static_cast<const bf16_t *>(weight), weight_row_stride, vocab,
      static_cast<bf16_t *>(out), out_row_stride, tokens, cpr);
  return wyh::launch_status();
}

extern "C" int wy_residual_add(const void *x, const void *residual, void *out, int64_t n,
                               void *stream) {
  if (!x || !residual || !out) return WY_E_NULL;
  if (n < 0) return WY_E_SHAPE;
  if (!wyh::aligned16(x) || !wyh::aligned16(residual) || !wyh::aligned16(out))
    return WY_E_LAYOUT;
  if (n == 0) return WY_OK;
  const int64_t threads = (n + 7) / 8;
  residual_add_kernel<<<unsigned((threads + 255) / 256), 256, 0,
                        static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(x), static_cast<const bf16_t *>(residual),
      static_cast<bf16_t *>(out), n);
  return wyh::launch_status();
}

extern "C" int wy_swiglu(const void *gate, const int64_t *gate_strides, const void *up,
                         const int64_t *up_strides, void *out, int rows, int cols,
                         void *stream) {
  if (!gate || !gate_strides || !up || !up_strides || !out) return WY_E_NULL;
  if (rows < 0 || cols < 0) return WY_E_SHAPE;
  if (rows == 0 || cols == 0) return WY_OK;
  const int vec = gate_strides[1] == 1 && up_strides[1] == 1 && cols % 8 == 0 &&
                  gate_strides[0] % 8 == 0 && up_strides[0] % 8 == 0 &&
                  wyh::aligned16(gate) && wyh::aligned16(up) && wyh::aligned16(out);
  const int64_t threads = vec ? int64_t(rows) * (cols / 8) : int64_t(rows) * cols;
  swiglu_kernel<<<unsigned((threads + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(gate), gate_strides[0], gate_strides[1],
      static_cast<const bf16_t *>(up), up_strides[0], up_strides[1], static_cast<bf16_t *>(out),
      rows, cols, vec);
  return wyh::launch_status();
}

extern "C" int64_t wy_lm_head_argmax_workspace_bytes(int rows, int hidden_size, int vocab) {
  if (rows <= 0 || hidden_size <= 0 || vocab <= 0) return 0;
  return int64_t(rows) * argmax_grid(rows, hidden_size, vocab) * 8;
}

extern "C" int wy_lm_head_argmax(const void *hidden, int64_t hidden_row_stride,
                                 const void *weight, int64_t weight_row_stride, int64_t *token_ids,
                                 int rows, int hidden_size, int vocab, void *workspace,
                                 int64_t workspace_bytes, void *stream) {
  if (!hidden || !weight || !token_ids || !workspace) return WY_E_NULL;
  if (rows <= 0 || rows > 64 || hidden_size <= 0 || vocab <= 0) return WY_E_SHAPE;
  if (hidden_size % (32 * kKBatch)) return WY_E_UNSUPPORTED;
  if (hidden_row_stride % 8 || weight_row_stride % 8 || !wyh::aligned16(hidden) ||
      !wyh::aligned16(weight) || (reinterpret_cast<uintptr_t>(workspace) & 7u))
    return WY_E_LAYOUT;
  if (workspace_bytes < wy_lm_head_argmax_workspace_bytes(rows, hidden_size, vocab))
    return WY_E_SHAPE;
  const int grid = argmax_grid(rows, hidden_size, vocab);
  const int mt = (rows + 15) / 16;
  const size_t lds = argmax_lds(rows, hidden_size);
  if (lds > 160 * 1024) return WY_E_SHAPE;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bf16_t *x = static_cast<const bf16_t *>(hidden);
  const bf16_t *w = static_cast<const bf16_t *>(weight);
  uint64_t *part = static_cast<uint64_t *>(workspace);
  int rc;
  switch (mt) {
    case 1: rc = launch_stage1<1>(grid, lds, st, x, hidden_row_stride, w, weight_row_stride, part,
                                  rows, hidden_size, vocab); break;
    case 2: rc = launch_stage1<2>(grid, lds, st, x, hidden_row_stride, w, weight_row_stride, part,
                                  rows, hidden_size, vocab); break;
    case 3: rc = launch_stage1<3>(grid, lds, st, x, hidden_row_stride, w, weight_row_stride, part,
                                  rows, hidden_size, vocab); break;
    default: rc = launch_stage1<4>(grid, lds, st, x, hidden_row_stride, w, weight_row_stride,
                                   part, rows, hidden_size, vocab); break;
  }
  if (rc != WY_OK) return rc;
  lm_head_argmax_stage2<<<rows, 64, 0, st>>>(part, grid, token_ids);
  return wyh::launch_status();
}
