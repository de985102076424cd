// y = x @ W^T in bf16 with fp32 accumulation on MFMA (gfx950): the projection
// GEMM of the attention block (triton_kernels/gemm_2d.py:157-240).
//   x [M, K], W [N, K], y [M, N]; K contiguous in x and W, N contiguous in y,
//   K % 128 == 0 (the reference's own precondition).
//
// Two kernels, chosen by M:
//   * M <= 64 (decode: M is the batch): weight streaming.  A workgroup owns 16
//     output columns (16 rows of W); its waves split K.  W rows are loaded
//     straight into the B operand of v_mfma_f32_16x16x32_bf16 (lane: column
//     l%16, 8 consecutive k at 8(l/16)), x rows into the A operand, one MFMA
//     per 16 rows of M, so every W byte is read once.  The waves' partial
//     16-column tiles are summed through LDS.
//   * M > 64 (prefill: M is the token count): 128 x 128 (4 waves of 64 x 64)
//     or 256 x 256 (8 waves of 128 x 64) output tiles on
//     v_mfma_f32_32x32x16_bf16, K in 64-wide steps.  x and W tiles move
//     global -> LDS with buffer loads carrying the LDS-DMA bit (no
//     registers), two stages; rows past M / N lie outside the buffer range
//     and read as zero.
#include <type_traits>

#include "wy_common.h"

using namespace wy;

namespace {

typedef float f32x4v_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

// ------------------------------------------------------------ skinny (M <= 64)
constexpr int kSkinnyMaxM = 64;
constexpr int kMaxSplit = 4;  // K splits across workgroups (skinny kernel)

// A-operand prologues of the skinny kernel (kPro):
//   0: A = x;
//   1: A = qwen_rmsnorm(x [+ residual]) = bf16(t * rsigma * (1 + w)) with
//      t = bf16(x + residual) (or x), rsigma from the same lane partition and
//      reduction order as qwen_rmsnorm_kernel; workgroup (0, 0) also writes t
//      to xout (the residual stream);
//   2: A = swiglu(x[:, :K], x[:, up_off:up_off+K]) = bf16(up * gate * sigmoid(gate)).
// Each equals the standalone kernels followed by the plain GEMM bit for bit.
struct ProArgs {
  const bf16_t *res;
  int64_t res0;
  const bf16_t *nw;
  float eps;
  bf16_t *xout;
  int64_t xo0;
  int64_t up_off;
};

__device__ __forceinline__ u32x4_t add_bf16x8(u32x4_t a, u32x4_t b) {
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = pack_bf16x2(bf16_lo(a[e]) + bf16_lo(b[e]), bf16_hi(a[e]) + bf16_hi(b[e]));
  return o;
}
__device__ __forceinline__ u32x4_t norm_bf16x8(u32x4_t t, float rs, u32x4_t w) {
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = pack_bf16x2(rms_apply(bf16_lo(t[e]), rs, bf16_lo(w[e])),
                       rms_apply(bf16_hi(t[e]), rs, bf16_hi(w[e])));
  return o;
}
__device__ __forceinline__ float swiglu_f(float g, float u) {
  return (u * g) * (1.0f / (1.0f + __expf(-g)));
}
__device__ __forceinline__ u32x4_t swiglu_bf16x8(u32x4_t g, u32x4_t u) {
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = pack_bf16x2(swiglu_f(bf16_lo(g[e]), bf16_lo(u[e])),
                       swiglu_f(bf16_hi(g[e]), bf16_hi(u[e])));
  return o;
}

// Gate/up-pair epilogue (kEpi 1): sums the waves' tiles of the gate and the
// up column tile in wave order, as the plain epilogue does, and stores
// bf16(swiglu(bf16(gate), bf16(up))).  With K split across workgroups the
// fp32 partials go to part[split][M][2N] (gate at column c, up at N + c)
// and the workgroup that completes cnt[blockIdx.x] sums them in split order.
template <int kNW, int kMT>
__device__ __forceinline__ void gate_up_epilogue(const f32x4v_t (&red)[kNW][kMT * 2][64],
                                 bf16_t *__restrict__ y, int64_t ys0, int M, int N, int n0,
                                 float *__restrict__ part, int32_t *__restrict__ cnt,
                                 int &last_ws) {
  const int n_split = int(gridDim.y);
  const int64_t pw = 2 * int64_t(N), part_stride = int64_t(M) * pw;
  for (int e = threadIdx.x; e < M * 16; e += 64 * kNW) {
    const int row = e >> 4, col = e & 15;
    const int mt = row >> 4, src = col + 16 * ((row & 15) >> 2), i = row & 3;
    float sg = 0.f, su = 0.f;
#pragma unroll
    for (int wv = 0; wv < kNW; ++wv) {
      sg += red[wv][mt * 2][src][i];
      su += red[wv][mt * 2 + 1][src][i];
    }
    if (n0 + col < N) {
      if (n_split == 1) {
        y[int64_t(row) * ys0 + n0 + col] = bf16_t(f32_to_bf16_bits(
            swiglu_f(round_bf16(sg), round_bf16(su))));
      } else {
        float *pp = part + blockIdx.y * part_stride + int64_t(row) * pw + n0 + col;
        __hip_atomic_store(pp, sg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pp + N, su, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (n_split == 1) return;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const int done = __hip_atomic_fetch_add(cnt + blockIdx.x, 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    const int last = done == n_split - 1;
    if (last) __hip_atomic_store(cnt + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_ws = last;
  }
  __syncthreads();
  if (!last_ws) return;
  for (int e = threadIdx.x; e < M * 16; e += 64 * kNW) {
    const int row = e >> 4, col = e & 15;
    if (n0 + col >= N) continue;
    const float *pp = part + int64_t(row) * pw + n0 + col;
    float g[kMaxSplit], u[kMaxSplit];
#pragma unroll
    for (int sp = 0; sp < kMaxSplit; ++sp) {
      const float *q = pp + (sp < n_split ? sp : 0) * part_stride;
      g[sp] = __hip_atomic_load(const_cast<float *>(q), __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
      u[sp] = __hip_atomic_load(const_cast<float *>(q + N), __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
    }
    float sg = 0.f, su = 0.f;
#pragma unroll
    for (int sp = 0; sp < kMaxSplit; ++sp) {
      sg += sp < n_split ? g[sp] : 0.f;
      su += sp < n_split ? u[sp] : 0.f;
    }
    y[int64_t(row) * ys0 + n0 + col] =
        bf16_t(f32_to_bf16_bits(swiglu_f(round_bf16(sg), round_bf16(su))));
  }
}

// Epilogues of the skinny kernel (kEpi):
//   0: y = bf16(acc);
//   1 (kNT == 2, gate/up pairs): the weight holds 2N rows, gate rows [0, N)
//      and up rows [N, 2N); a workgroup's column tile 0 covers gate rows
//      n0..n0+15 and tile 1 the up rows N+n0..; y[:, n0 + c] =
//      bf16(swiglu(bf16(gate acc), bf16(up acc))), the [M, N] SwiGLU output
//      of the [M, 2N] projection, equal to the plain GEMM followed by
//      swiglu_kernel whenever the plain GEMM's plan matches (same waves and
//      K split; 2N >= 4096).
template <int kNW, int kMT, int kNT, int kPro = 0, int kEpi = 0>
__global__ __launch_bounds__(64 * kNW) void gemm_skinny_kernel(
    const bf16_t *__restrict__ x, int64_t xs0, const bf16_t *__restrict__ w, int64_t ws0,
    bf16_t *__restrict__ y, int64_t ys0, int M, int N, int K, float *__restrict__ part,
    int32_t *__restrict__ cnt, const ProArgs pro) {
  // kMT = ceil(M / 16) tiles of 16 rows, kNT tiles of 16 columns per
  // workgroup (each x load feeds kNT MFMAs); every load of a 4-step batch is
  // issued before the first MFMA consumes one, so a wave waits for memory once
  // per 128 columns of K rather than once per load.
  // Split K (gridDim.y > 1): workgroup (x, y) sums K range y of gridDim.y,
  // publishes its fp32 tile to part[y] and counts itself on cnt[x]; the
  // workgroup that completes the count adds the tiles in split order (so the
  // result does not depend on which one arrives last), stores bf16 and
  // resets the counter.
  __shared__ f32x4v_t red[kNW][kMT * kNT][64];
  __shared__ int last_ws;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  static_assert(kEpi == 0 || kNT == 2, "gate/up pairs need two column tiles");
  const int n0 = blockIdx.x * 16 * (kEpi == 1 ? 1 : kNT);
  const int n_split = int(gridDim.y);
  const int ks = K / n_split;  // a multiple of 32 * kNW (host)
  const int kc = ks / kNW;
  const int kb = int(blockIdx.y) * ks + wave * kc;
  const int g = lane >> 4;
  const bf16_t *wp[kNT];
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt)
    wp[nt] = w +
             (kEpi == 1 ? int64_t(min(n0 + (lane & 15), N - 1)) + int64_t(nt) * N
                        : int64_t(min(n0 + 16 * nt + (lane & 15), N - 1))) * ws0 +
             kb + 8 * g;
  const bf16_t *xp[kMT];
  bool xok[kMT];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) {
    const int row = mt * 16 + (lane & 15);
    xok[mt] = row < M;
    xp[mt] = x + int64_t(xok[mt] ? row : 0) * xs0 + kb + 8 * g;
  }
  // K runs in batches of four 32-wide steps (all loads of a batch issued
  // before its first MFMA), then one batch of the remaining kc % 128 steps,
  // loaded together as well.  The first full batch's W rows are requested
  // before the A prologue, which does not need them.
  const int nfull = kc >> 7, rem = (kc & 127) >> 5;
  u32x4_t w_first[4][kNT];
  if (nfull > 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) w_first[j][nt] = ld16(wp[nt] + 32 * j);
  }
  float rsr[kMT];
  const bf16_t *rp[kMT];
  const bf16_t *nwp = nullptr;
  if constexpr (kPro == 1) {
    // rsigma of every row: 32 lanes per row, lane l summing the 8-element
    // chunks (32 kk + l) * 8 in order, then the xor tree (rms_rsigma)
    __shared__ float rs_lds[kSkinnyMaxM];
    const int l32 = threadIdx.x & 31;
    const bool write_x = pro.xout && blockIdx.x == 0 && blockIdx.y == 0;
    for (int row = threadIdx.x >> 5; row < M; row += 2 * kNW) {
      const bf16_t *hr = x + int64_t(row) * xs0;
      const bf16_t *rr = pro.res ? pro.res + int64_t(row) * pro.res0 : nullptr;
      float ss = 0.f;
      for (int kk = 0; kk < K / 256; ++kk) {
        const int c = (32 * kk + l32) * 8;
        u32x4_t t = ld16(hr + c);
        if (rr) t = add_bf16x8(t, ld16(rr + c));
        if (write_x) st16(pro.xout + int64_t(row) * pro.xo0 + c, t);
        ss = rms_acc8(t, ss);
      }
      const float rs = rms_rsigma(ss, K, pro.eps);
      if (l32 == 0) rs_lds[row] = rs;
    }
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt) {
      const int row = mt * 16 + (lane & 15);
      rsr[mt] = xok[mt] ? rs_lds[row] : 0.f;
      rp[mt] = pro.res ? pro.res + int64_t(xok[mt] ? row : 0) * pro.res0 + kb + 8 * g : nullptr;
    }
    nwp = pro.nw + kb + 8 * g;
  }
  // the A operand of rows tile mt at k offset kk (relative to kb + 8 g)
  auto load_a = [&](int mt, int kk) -> u32x4_t {
    u32x4_t v = ld16(xp[mt] + kk);
    if constexpr (kPro == 1) {
      if (rp[mt]) v = add_bf16x8(v, ld16(rp[mt] + kk));
      v = norm_bf16x8(v, rsr[mt], ld16(nwp + kk));
    } else if constexpr (kPro == 2) {
      v = swiglu_bf16x8(v, ld16(xp[mt] + pro.up_off + kk));
    }
    return v;
  };
  f32x4v_t acc[kMT][kNT];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) acc[mt][nt] = f32x4v_t{0.f, 0.f, 0.f, 0.f};
  auto step = [&](const u32x4_t (&wv)[kNT], u32x4_t xv, int mt) {
    if (!xok[mt]) xv = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
      acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8_t, xv), __builtin_bit_cast(bf16x8_t, wv[nt]), acc[mt][nt], 0,
          0, 0);
  };
  // R steps from k: x loads, then the MFMAs over the given W rows
  auto batch = [&](auto steps, const u32x4_t (&wv)[decltype(steps)::value][kNT], int k) {
    constexpr int R = decltype(steps)::value;
    u32x4_t xv[kMT][R];
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int j = 0; j < R; ++j) xv[mt][j] = load_a(mt, k + 32 * j);
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt) step(wv[j], xv[mt][j], mt);
  };
  auto load_batch = [&](auto steps, int k) {
    constexpr int R = decltype(steps)::value;
    u32x4_t wv[R][kNT];
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) wv[j][nt] = ld16(wp[nt] + k + 32 * j);
    batch(steps, wv, k);
  };
  using S4 = std::integral_constant<int, 4>;
  if (nfull > 0) batch(S4{}, w_first, 0);
  for (int b = 1; b < nfull; ++b) load_batch(S4{}, 128 * b);
  const int kt = 128 * nfull;
  if (rem == 1) load_batch(std::integral_constant<int, 1>{}, kt);
  else if (rem == 2) load_batch(std::integral_constant<int, 2>{}, kt);
  else if (rem == 3) load_batch(std::integral_constant<int, 3>{}, kt);

  // lane l of tile (mt, nt) holds rows mt*16 + 4(l/16) + i (i = 0..3) of
  // column 16 nt + l%16
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) red[wave][mt * kNT + nt][lane] = acc[mt][nt];
  __syncthreads();
  if constexpr (kEpi == 1) {
    gate_up_epilogue<kNW, kMT>(red, y, ys0, M, N, n0, part, cnt, last_ws);
    return;
  }
  const int64_t part_stride = int64_t(M) * N;
  for (int e = threadIdx.x; e < M * 16 * kNT; e += 64 * kNW) {
    const int row = e / (16 * kNT), cc = e - row * (16 * kNT);
    const int nt = cc >> 4, col = cc & 15;
    const int mt = row >> 4, src = col + 16 * ((row & 15) >> 2), i = row & 3;
    float s = 0.f;
#pragma unroll
    for (int wv = 0; wv < kNW; ++wv) s += red[wv][mt * kNT + nt][src][i];
    if (n0 + cc < N) {
      if (n_split == 1)
        y[int64_t(row) * ys0 + n0 + cc] = bf16_t(f32_to_bf16_bits(s));
      else  // device-coherent: another workgroup (maybe on another XCD) reads it
        __hip_atomic_store(part + blockIdx.y * part_stride + int64_t(row) * N + n0 + cc, s,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (n_split == 1) return;
  // The partial stores have completed before the count (a workgroup-scope
  // fence alone does not wait for them).
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const int done = __hip_atomic_fetch_add(cnt + blockIdx.x, 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    const int last = done == n_split - 1;
    if (last) __hip_atomic_store(cnt + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_ws = last;
  }
  __syncthreads();
  if (!last_ws) return;
  // Every partial of every element this thread sums is requested before the
  // first is added (one memory round trip); splits past n_split read split 0
  // and weigh 0.
  constexpr int kPer = (kSkinnyMaxM * 16 * kNT + 64 * kNW - 1) / (64 * kNW);
  float v[kPer][kMaxSplit];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int e = threadIdx.x + u * 64 * kNW;
    const int row = e / (16 * kNT), cc = e - row * (16 * kNT);
    const bool ok = e < M * 16 * kNT && n0 + cc < N;
    const float *pp = part + (ok ? int64_t(row) * N + n0 + cc : 0);
#pragma unroll
    for (int sp = 0; sp < kMaxSplit; ++sp)
      v[u][sp] = __hip_atomic_load(const_cast<float *>(pp + (sp < n_split ? sp : 0) * part_stride),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int e = threadIdx.x + u * 64 * kNW;
    const int row = e / (16 * kNT), cc = e - row * (16 * kNT);
    if (e >= M * 16 * kNT || n0 + cc >= N) continue;
    float s = 0.f;
#pragma unroll
    for (int sp = 0; sp < kMaxSplit; ++sp) s += sp < n_split ? v[u][sp] : 0.f;
    y[int64_t(row) * ys0 + n0 + cc] = bf16_t(f32_to_bf16_bits(s));
  }
}

// ------------------------------------------------------------ tiled (M > 64)
// Output tile BM x BN, WM x WN waves of (BM/WM) x (BN/WN) as 32 x 32 MFMA
// tiles; K in 64-wide steps through an LDS ring of kS stages (two, or four
// for a grid of at most one workgroup per CU) filled by LDS-DMA buffer loads
// (rows past M / N lie outside the buffer range and read zero).
// The MFMA operands are read from LDS with explicit waits: the reads of
// k-step ks+1 are issued before the MFMAs of ks and awaited after them, so
// the LDS latency hides behind the MFMAs (left to the compiler, each read
// pair was awaited right before its MFMA).
//   <128, 128, 2, 2>: 64 KiB of LDS (swizzled rows), two workgroups per CU;
//   <256, 256, 2, 4>: 8 waves of 128 x 64, 128 KiB, one workgroup per CU --
//   half the LDS bytes per MFMA; used when the grid fills the chip.

// One 1 KiB global -> LDS block (16 bytes per lane).  A plain device function:
// inside a kernel template the host-side pass cannot instantiate the builtin.
__device__ __forceinline__ void dma_block(__amdgpu_buffer_rsrc_t rsrc, unsigned char *lds,
                                          uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t *)lds, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ uint32_t lds_u32(const unsigned char *p) {
  return uint32_t(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) unsigned char *)(p)));
}
// ds_read_b128 as asm: the compiler does not track it, the caller awaits it
// with lgkm_wait_all, whose "+v" operands keep later uses after the wait.
template <int kOff>
__device__ __forceinline__ u32x4_t ds_read16(uint32_t addr) {
  u32x4_t r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(kOff));
  return r;
}
template <int kFM, int kFN>
__device__ __forceinline__ void lgkm_wait_all(u32x4_t (&a)[kFM], u32x4_t (&b)[kFN]) {
  if constexpr (kFM == 2 && kFN == 2)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]));
  else if constexpr (kFM == 2 && kFN == 1)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]));
  else if constexpr (kFM == 4 && kFN == 1)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]));
  else if constexpr (kFM == 4 && kFN == 2)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]));
  else
    static_assert(kFM < 0, "fragment counts without a wait");
}
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// LDS row layout of a stage: a tile row holds its 64 k values (128 bytes, no
// pad slot) with 16-byte chunk c in slot c ^ swz(r).  Two rows share a
// 256-byte line of the 64 banks, and swz(r) = (r / 2) % 8 makes the 16 rows
// that a quarter-wave of ds_read_b128 touches fill all 16 slots of the line
// (swizzling on r % 8 left every read 2-way conflicted; a pad slot per row
// costs 1/9 more LDS per stage).
constexpr int kTK = 64;  // k values per ring stage
struct TileRows {
  static constexpr int kChunks = kTK / 8;  // 16-byte chunks of k per row
  static constexpr int kPitch = kChunks * 16;
  static constexpr int kRowsPerLine = 256 / kPitch;
  __device__ static constexpr int swz(int row) { return (row / kRowsPerLine) % kChunks; }
};

template <int BM, int BN, int WM, int WN, int kS = 2>
struct TileCfg {
  using R = TileRows;
  static constexpr int kWaves = WM * WN;
  static constexpr int kATile = BM * R::kPitch, kBTile = BN * R::kPitch;
  static constexpr int kStage = kATile + kBTile;
  static constexpr int kABlk = kATile / 1024;           // DMA blocks of the x tile
  static constexpr int kBlk = kABlk + kBTile / 1024;     // DMA blocks per stage
  static constexpr int kPerWave = (kBlk + kWaves - 1) / kWaves;
  static constexpr int kLds = kS * kStage;  // a ring of kS stages
  static constexpr int kFM = BM / WM / 32, kFN = BN / WN / 32;  // MFMA tiles per wave
  static_assert(kATile % 1024 == 0 && kBTile % 1024 == 0, "whole DMA blocks");
};

// Output tile of workgroup L (a 1-D grid of tm * tn tiles).  Workgroups are
// dealt to the 8 XCDs round-robin (L % 8), each XCD with its own L2; XCD x
// takes a contiguous range of the tile order, and that order walks groups of
// gm M-tiles column by column, so the workgroups an XCD runs together share
// their x rows and W rows in that XCD's L2 instead of every XCD fetching
// every tile's operands.
constexpr int kXcds = 8;
__device__ __forceinline__ void tile_of(int L, int tm, int tn, int gm, int &mt, int &nt) {
  const int T = tm * tn;
  const int per = (T + kXcds - 1) / kXcds;      // tiles of the fuller XCDs
  const int full = T - kXcds * (per - 1);       // XCDs holding `per` tiles
  const int x = L % kXcds, i = L / kXcds;
  const int t = x < full ? x * per + i : full * per + (x - full) * (per - 1) + i;
  const int grp = gm * tn;
  const int first_m = (t / grp) * gm;
  const int gsz = min(tm - first_m, gm);
  const int r = t - (t / grp) * grp;
  mt = first_m + r % gsz;
  nt = r / gsz;
}

// kSwiGLU (gate/up pairs): w holds 2N rows, gate rows [0, N) and up rows
// [N, 2N), and a tile spans BN/2 output columns: each wave's first 32-column
// MFMA tile loads the gate rows of its 32 columns, its second the up rows of
// the same columns, so a lane holds gate and up of one output element and the
// epilogue writes y [M, N] = bf16(swiglu(bf16(gate), bf16(up))).
template <int BM, int BN, int WM, int WN, bool kSwiGLU = false, int kS = 2>
__global__ __launch_bounds__(64 * WM * WN) void gemm_tiled_kernel(
    const bf16_t *__restrict__ x, int64_t xs0, const bf16_t *__restrict__ w, int64_t ws0,
    bf16_t *__restrict__ y, int64_t ys0, int M, int N, int K, int gm) {
  using C = TileCfg<BM, BN, WM, WN, kS>;
  using R = typename C::R;
  constexpr int kTPitch = R::kPitch;
  static_assert(!kSwiGLU || BN / WN == 64, "gate/up pairs: two 32-column tiles per wave");
  constexpr int kOutBN = kSwiGLU ? BN / 2 : BN;  // output columns per tile
  constexpr int kFM = C::kFM, kFN = C::kFN;
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int g = lane >> 5, r32 = lane & 31;
  int mt, nt;
  tile_of(int(blockIdx.x), (M + BM - 1) / BM, (N + kOutBN - 1) / kOutBN, gm, mt, nt);
  const int m0 = mt * BM, n0 = nt * kOutBN;

  // DMA block b (= wave + kWaves*i) of a stage: b < kABlk fills the x tile,
  // the rest the W tile; lane j of a block fills 16-byte slot 64 (b mod
  // tile) + j; slot c of row r holds k-chunk c (the pad slot repeats chunk
  // 0, never read).  Lane offsets are tile-invariant, the k offset is scalar,
  // and the buffer ranges end at the last valid row.
  const int a_rows = min(BM, M - m0), b_rows = min(BN, N - n0);
  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t *>(x + int64_t(m0) * xs0), 0,
      int(uint32_t(a_rows - 1) * uint32_t(xs0) * 2u + uint32_t(K) * 2u), 0x00020000);
  // gate/up pairs: the W buffer is the whole [2N, K] matrix (N % kOutBN == 0,
  // host), tile row r -> W row (r % 64 < 32 ? 0 : N) + n0 + 32 (r / 64) + r % 32
  const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t *>(kSwiGLU ? w : w + int64_t(n0) * ws0), 0,
      kSwiGLU ? int(uint32_t(2 * N - 1) * uint32_t(ws0) * 2u + uint32_t(K) * 2u)
              : int(uint32_t(b_rows - 1) * uint32_t(ws0) * 2u + uint32_t(K) * 2u),
      0x00020000);
  uint32_t voff[C::kPerWave];
#pragma unroll
  for (int i = 0; i < C::kPerWave; ++i) {
    const int blk = min(wave + C::kWaves * i, C::kBlk - 1);
    const bool is_a = blk < C::kABlk;
    const int sl = 64 * (is_a ? blk : blk - C::kABlk) + lane;
    const int row = sl / R::kChunks, c = sl - (sl / R::kChunks) * R::kChunks;
    const uint32_t cb =
        uint32_t(c ^ R::swz(row)) * 16u;
    int wrow = row;
    if (kSwiGLU && !is_a)
      wrow = ((row & 63) < 32 ? 0 : N) + n0 + 32 * (row >> 6) + (row & 31);
    voff[i] = uint32_t(wrow) * uint32_t(is_a ? xs0 : ws0) * 2u + cb;
  }
  // With more than two stages every wave issues exactly kPerWave DMAs per
  // stage (a wave past the last block repeats it: the same bytes to the same
  // LDS slot), so that the wait for the oldest stage is a fixed count of the
  // wave's younger loads.
  auto issue = [&](int kt, int i0 = 0, int i1 = C::kPerWave) {
    unsigned char *st = smem + (kt % kS) * C::kStage;
    const uint32_t soff = uint32_t(kt * kTK) * 2u;
#pragma unroll
    for (int i = 0; i < C::kPerWave; ++i) {
      if (i < i0 || i >= i1) continue;
      const int blk0 = wave + C::kWaves * i;  // wave-uniform
      if constexpr (C::kABlk % C::kWaves == 0 && C::kBlk % C::kWaves == 0) {
        // block i of every wave is an x block for i < kABlk / kWaves: no branch
        dma_block(i < C::kABlk / C::kWaves ? a_rsrc : b_rsrc, st + blk0 * 1024, voff[i], soff);
      } else {
        if (kS == 2 && blk0 >= C::kBlk) continue;
        const int blk = min(blk0, C::kBlk - 1);
        if (blk < C::kABlk) dma_block(a_rsrc, st + blk * 1024, voff[i], soff);
        else dma_block(b_rsrc, st + blk * 1024, voff[i], soff);
      }
    }
  };

  f32x16_t acc[kFM][kFN];
#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int j = 0; j < kFN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int kt_n = K / kTK;
#pragma unroll
  for (int s0 = 0; s0 + 1 < kS; ++s0)
    if (s0 < kt_n) issue(s0);
  // lane address of k sub-step ks's chunk (2 ks + g) in the wave's first
  // row (r32); rows 32 apart share the swizzle
  static_assert(32 % (R::kRowsPerLine * R::kChunks) == 0, "swizzle period");
  uint32_t a_lane[kTK / 16], b_lane[kTK / 16];
#pragma unroll
  for (int ks = 0; ks < kTK / 16; ++ks) {
    const uint32_t cs = uint32_t(16 * ((2 * ks + g) ^ R::swz(r32)));
    a_lane[ks] = uint32_t((BM / WM * wm + r32) * kTPitch) + cs;
    b_lane[ks] = uint32_t(C::kATile + (BN / WN * wn + r32) * kTPitch) + cs;
  }
  // wait until stage t has landed: the wave's loads younger than it are the
  // stages t + 1 .. t + kS - 2 that were issued (fewer near the end of K)
  auto wait_stage = [&](int t) {
    if constexpr (kS == 2) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
      static_assert((kS - 2) * C::kPerWave <= 63, "vmcnt range");
      if (t + kS - 2 < kt_n)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((kS - 2) * C::kPerWave) : "memory");
      else if (kS == 4 && t + 1 < kt_n)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(C::kPerWave) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
  };
  // A bare s_barrier: __syncthreads' workgroup release fence would also wait
  // for every DMA in flight (vmcnt(0)), which collapses the ring to one stage.
  auto barrier = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  u32x4_t av[2][kFM], bv[2][kFN];
  auto load = [&](uint32_t st, auto bufc, auto ksc) {
    constexpr int buf = decltype(bufc)::value, ks = decltype(ksc)::value;
    const uint32_t abase = st + a_lane[ks], bbase = st + b_lane[ks];
    static_for<0, kFM>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
      av[buf][t] = ds_read16<t * 32 * kTPitch>(abase);
    });
    static_for<0, kFN>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
      bv[buf][t] = ds_read16<t * 32 * kTPitch>(bbase);
    });
  };
// The MFMA batch runs at raised wave priority (s_setprio), so the wave that
// has operands keeps the matrix pipe fed while the SIMD's other wave issues
// its LDS reads and DMA (1-4% on every tile shape).
  auto mfmas = [&](auto bufc) {
    constexpr int cur = decltype(bufc)::value;
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int i = 0; i < kFM; ++i)
#pragma unroll
      for (int j = 0; j < kFN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, av[cur][i]), __builtin_bit_cast(bf16x8_t, bv[cur][j]),
            acc[i][j], 0, 0, 0);
    __builtin_amdgcn_s_setprio(0);
  };
  const uint32_t smem0 = lds_u32(smem);
  constexpr int kKS = kTK / 16;  // MFMA k sub-steps per stage (even)
  static_assert(kKS % 2 == 0, "sub-step buffers alternate");
  if constexpr (C::kWaves == 4 || kS > 2) {
    // split of a stage's DMA: the first part right after the barrier, the
    // rest after the next step's first sub-step (8-wave tile)
    constexpr int kHalf = C::kWaves == 8 ? (C::kPerWave + 1) / 2 : C::kPerWave;
    // The barrier that hands slot kt back to the DMA and makes stage kt + 1
    // visible sits before the last sub-step of step kt: the reads of step
    // kt + 1's first sub-step and the refill DMA then overlap that sub-step's
    // MFMAs instead of opening every step with an exposed LDS round trip
    // (4-wave tiles 2-5% faster, the 8-wave 4-stage tile 5%, with its DMA
    // split around the barrier; the 8-wave 2-stage 256 x 256 tile keeps a
    // barrier that opens the step and its DMA spread over the first two
    // sub-steps, 1-3% better there).
    wait_stage(0);
    barrier();
    load(smem0, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    if (kS - 1 < kt_n) issue(kS - 1);
    for (int kt = 0; kt < kt_n; ++kt) {
      const uint32_t st = smem0 + uint32_t((kt % kS) * C::kStage);
      const bool more = kt + 1 < kt_n;
      lgkm_wait_all<kFM, kFN>(av[0], bv[0]);
      static_for<0, kKS>([&](auto ksc) {
        constexpr int ks = decltype(ksc)::value, cur = ks & 1;
        if constexpr (ks + 1 < kKS) {
          load(st, std::integral_constant<int, cur ^ 1>{}, std::integral_constant<int, ks + 1>{});
        } else {
          if (more) {
            wait_stage(kt + 1);
            barrier();
            load(smem0 + uint32_t(((kt + 1) % kS) * C::kStage),
                 std::integral_constant<int, cur ^ 1>{}, std::integral_constant<int, 0>{});
            if (kt + kS < kt_n) issue(kt + kS, 0, kHalf);
            // keep this sub-step's MFMAs after the barrier (they touch no
            // memory, so the compiler would otherwise hoist them above it)
            u32x4_t(&ac)[kFM] = av[cur];
            u32x4_t(&bc)[kFN] = bv[cur];
#pragma unroll
            for (int t = 0; t < kFM; ++t) asm volatile("" : "+v"(ac[t]));
#pragma unroll
            for (int t = 0; t < kFN; ++t) asm volatile("" : "+v"(bc[t]));
          }
        }
        mfmas(std::integral_constant<int, cur>{});
        if constexpr (ks == 0 && kHalf < C::kPerWave)
          if (kt >= 1 && kt - 1 + kS < kt_n) issue(kt - 1 + kS, kHalf, C::kPerWave);
        if constexpr (ks + 1 < kKS) lgkm_wait_all<kFM, kFN>(av[cur ^ 1], bv[cur ^ 1]);
      });
    }
  } else {
  for (int kt = 0; kt < kt_n; ++kt) {
    wait_stage(kt);
    barrier();  // and every wave is done with the slot refilled next
    // the next stage's DMA blocks: issued together after the barrier, or for
    // the 8-wave two-stage tile spread over the first two k-steps (fewer LDS
    // writes landing while all waves read their first operands: 256 x 256
    // shapes 3-6% faster, the 4-wave tiles slower)
    constexpr int kSpread = C::kWaves == 8 && kS == 2 ? 2 : 1;
    constexpr int kPerStep = (C::kPerWave + kSpread - 1) / kSpread;
    const bool more = kt + kS - 1 < kt_n;
    if (more) issue(kt + kS - 1, 0, kPerStep);
    const uint32_t st = smem0 + uint32_t((kt % kS) * C::kStage);
    load(st, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    lgkm_wait_all<kFM, kFN>(av[0], bv[0]);
    static_for<0, kKS>([&](auto ksc) {
      constexpr int ks = decltype(ksc)::value, cur = ks & 1;
      if constexpr (ks + 1 < kKS)
        load(st, std::integral_constant<int, cur ^ 1>{}, std::integral_constant<int, ks + 1>{});
      mfmas(std::integral_constant<int, cur>{});
      if constexpr (ks + 1 < kSpread)
        if (more) issue(kt + kS - 1, (ks + 1) * kPerStep, (ks + 2) * kPerStep);
      if constexpr (ks + 1 < kKS) lgkm_wait_all<kFM, kFN>(av[cur ^ 1], bv[cur ^ 1]);
    });
  }
  }

  // acc[i][j] register r of lane l: row (r&3) + 8(r>>2) + 4(l/32) of m-tile i,
  // column l%32 of n-tile j.  With 16-byte-aligned output rows each wave
  // stages its sub-tile in LDS (the ring is free once every wave is past its
  // last operand read) and writes whole 16-byte pieces of its rows with
  // non-temporal stores; otherwise element by element.
  if constexpr (kSwiGLU) {
    // lane: output column 32 wn + r32 of the tile's BN/2, rows 32 i + (r&3) +
    // 8(r>>2) + 4g of the wave's 128; the whole BM x BN/2 output tile is
    // staged in LDS, then stored as whole row pieces by all waves
    constexpr int kRWs = BM / WM, kSPs = kOutBN * 2 + 16;
    static_assert(BM * kSPs <= C::kLds, "output stage fits the ring");
    __syncthreads();
    // rows r, r + 1 of columns c, c + 1 as one bf16 pair per lane, exchanged
    // between adjacent lanes as in the plain epilogue below
    const bool odd = lane & 1;
#pragma unroll
    for (int i = 0; i < kFM; ++i)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float a0 = swiglu_f(round_bf16(acc[i][0][r]), round_bf16(acc[i][1][r]));
        const float a1 = swiglu_f(round_bf16(acc[i][0][r + 1]), round_bf16(acc[i][1][r + 1]));
        const float recv = __int_as_float(__builtin_amdgcn_update_dpp(
            0, __float_as_int(odd ? a0 : a1), 0xB1, 0xf, 0xf, false));  // quad_perm [1,0,3,2]
        const int row = kRWs * wm + 32 * i + (r & 3) + 8 * (r >> 2) + 4 * g + (odd ? 1 : 0);
        *reinterpret_cast<uint32_t *>(smem + row * kSPs + (32 * wn + (r32 & ~1)) * 2) =
            odd ? pack_bf16x2(recv, a1) : pack_bf16x2(a0, recv);
      }
    __syncthreads();
    const bool vec = ((N | ys0) & 7) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    constexpr int kCPR = kOutBN / 8;  // 16-byte pieces per row
#pragma unroll 4
    for (int e = threadIdx.x; e < BM * kCPR; e += 64 * C::kWaves) {
      const int row = e / kCPR, c = e - row * kCPR;
      const int grow = m0 + row, gcol = n0 + 8 * c;
      if (grow >= M) continue;
      const u32x4_t v = ld16(smem + row * kSPs + 16 * c);
      bf16_t *dst = y + int64_t(grow) * ys0 + gcol;
      if (vec) {
        st16_nt(dst, v);
      } else {
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          dst[2 * h] = bf16_t(v[h] & 0xffffu);
          dst[2 * h + 1] = bf16_t(v[h] >> 16);
        }
      }
    }
    return;
  }
  constexpr int kRW = BM / WM, kCW = BN / WN;   // the wave's sub-tile
  constexpr int kSP = kCW * 2 + 16;             // staged row pitch, bytes
  const bool vec_out = ((N | ys0) & 7) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
  if (vec_out) {
    // The ring slot the last K step did not use is free once every wave is
    // past the last step's barrier (no DMA targets it any more), so each wave
    // stages its sub-tile there without another barrier: in kParts row
    // bands when the whole sub-tile does not fit, each band read back before
    // the next is written (one wave's LDS operations complete in order).
    // (when no band of whole MFMA tiles fits one slot, all waves first meet
    // at a barrier and the bands go to the whole ring)
    constexpr auto fits = [](int parts, int room) {
      return kFM % parts == 0 && C::kWaves * (kRW / parts) * kSP <= room;
    };
    constexpr bool kInSlot = fits(1, C::kStage) || fits(2, C::kStage) || fits(4, C::kStage);
    constexpr int kRoom = kInSlot ? C::kStage : C::kLds;
    constexpr int kParts = fits(1, kRoom) ? 1 : fits(2, kRoom) ? 2 : 4;
    static_assert(fits(kParts, kRoom), "output band fits");
    if constexpr (!kInSlot) __syncthreads();
    unsigned char *const stg = smem + (kInSlot ? (kt_n % kS) * C::kStage : 0) +
                               wave * ((kRW / kParts) * kSP);
    // rows r, r + 1 (r even) of columns c, c + 1 (c even) sit in lanes c and
    // c + 1; one DPP swap of adjacent lanes gives the even lane row r and the
    // odd lane row r + 1 of both columns, written as one bf16 pair (half the
    // LDS writes of 2-byte stores, and no two lanes share a dword)
    const bool odd = lane & 1;
    constexpr int kCPR = kCW / 8;   // 16-byte pieces per row
#pragma unroll
    for (int part = 0; part < kParts; ++part) {
#pragma unroll
      for (int ii = 0; ii < kFM / kParts; ++ii) {
        const int i = part * (kFM / kParts) + ii;
#pragma unroll
        for (int j = 0; j < kFN; ++j)
#pragma unroll
          for (int r = 0; r < 16; r += 2) {
            const float a0 = acc[i][j][r], a1 = acc[i][j][r + 1];
            const float recv = __int_as_float(__builtin_amdgcn_update_dpp(
                0, __float_as_int(odd ? a0 : a1), 0xB1, 0xf, 0xf, false));  // quad_perm [1,0,3,2]
            const int row = 32 * ii + (r & 3) + 8 * (r >> 2) + 4 * g + (odd ? 1 : 0);
            *reinterpret_cast<uint32_t *>(stg + row * kSP + (32 * j + (r32 & ~1)) * 2) =
                odd ? pack_bf16x2(recv, a1) : pack_bf16x2(a0, recv);
          }
      }
      constexpr int kBandRows = kRW / kParts;
#pragma unroll 4
      for (int e = lane; e < kBandRows * kCPR; e += 64) {
        const int row = e / kCPR, c = e - row * kCPR;
        const int grow = m0 + kRW * wm + part * kBandRows + row, gcol = n0 + kCW * wn + 8 * c;
        if (grow < M && gcol < N)
          st16_nt(y + int64_t(grow) * ys0 + gcol, ld16(stg + row * kSP + 16 * c));
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int j = 0; j < kFN; ++j) {
      const int col = n0 + BN / WN * wn + 32 * j + r32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + BM / WM * wm + 32 * i + (r & 3) + 8 * (r >> 2) + 4 * g;
        if (row < M && col < N)
          y[int64_t(row) * ys0 + col] = bf16_t(f32_to_bf16_bits(acc[i][j][r]));
      }
    }
}

#ifndef WY_GEMM_GROUP_M
#define WY_GEMM_GROUP_M 4
#endif
template <int BM, int BN, int WM, int WN, bool kSwiGLU = false, int kS = 2>
int launch_tiled_cfg(const bf16_t *x, int64_t xs0, const bf16_t *w, int64_t ws0, bf16_t *y,
                     int64_t ys0, int M, int N, int K, hipStream_t st) {
  using C = TileCfg<BM, BN, WM, WN, kS>;
  static_assert(C::kLds <= 160 * 1024, "LDS");
  auto *fn = gemm_tiled_kernel<BM, BN, WM, WN, kSwiGLU, kS>;
  // once per instantiation; a function-local static is initialised exactly
  // once, also under concurrent first calls
  static const hipError_t attr_rc = hipFuncSetAttribute(
      reinterpret_cast<const void *>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, C::kLds);
  if (attr_rc != hipSuccess) return int(attr_rc);
  const int tm = (M + BM - 1) / BM, tn = (N + (kSwiGLU ? BN / 2 : BN) - 1) / (kSwiGLU ? BN / 2 : BN);
  fn<<<unsigned(tm * tn), 64 * C::kWaves, C::kLds, st>>>(x, xs0, w, ws0, y, ys0, M, N, K,
                                                         WY_GEMM_GROUP_M);
  return wyh::launch_status();
}

// The 256 x 256 tile from 384 of its tiles (a round and a half of the 256 CUs,
// one workgroup each: the 4096-token in_proj / gate_up shapes 115 -> 102 and
// 73 -> 68 us; at 320 tiles, [4096, 5120], it lost 54 -> 65 us), else 128 x
// 128 (two workgroups per CU, four times the workgroups, so a partial last
// round costs less), or 128 x 64 below two 128 x 128 tiles per CU.
// Tile shape and ring depth per grid (every variant swizzles its LDS rows and
// steps K by 64; 32-wide K steps measured slower on every shape):
//   256 x 256, 2 stages: from 384 tiles, or when 240..256 tiles make one
//     round of the 256 CUs (the 3 stages a deeper ring needs do not fit);
//   128 x 64, 4 stages: at most 256 such tiles, i.e. at most one workgroup
//     per CU, where nothing else hides the latency (k_proj at 4096 tokens);
//   128 x 128 on 8 waves (64 x 32 each), 4 stages: fewer than two 128 x 128
//     tiles per CU but more than one round of 128 x 64 ones (o_proj and
//     down_proj at 4096 tokens: one workgroup per CU with a deep ring beat
//     two per CU with two stages, and 8 waves beat 4 there: o_proj 22.4 ->
//     20.1 us);
//   128 x 128, 2 stages: otherwise (two workgroups per CU; a deeper ring
//     would cost the second one).
constexpr int kBigMinTiles = 384, kBigRoundTiles = 240, kCUs = 256;
int launch_tiled(const bf16_t *x, int64_t xs0, const bf16_t *w, int64_t ws0, bf16_t *y,
                 int64_t ys0, int M, int N, int K, hipStream_t st) {
  const int64_t big = int64_t((M + 255) / 256) * ((N + 255) / 256);
  const bool use_big = big >= kBigMinTiles || (big >= kBigRoundTiles && big <= kCUs);
  // A narrow last column of 256-wide tiles (N % 256 <= 64, e.g. the GDN
  // in_proj's 8224 = 8192 + 32) costs a whole extra round of tiles for a
  // few columns: those columns run as a second, narrow launch (each output
  // element's K order is the same in every tile shape, so the result is
  // unchanged; 4096 x 8224: 90.5 -> 68.1 + 9.2 us).
  const int tail = N % 256;
  if (use_big && tail != 0 && tail <= 64 && N > 256) {
    const int n_main = N - tail;
    const int rc = launch_tiled_cfg<256, 256, 2, 4, false, 2>(x, xs0, w, ws0, y, ys0,
                                                                       M, n_main, K, st);
    if (rc != WY_OK) return rc;
    return launch_tiled(x, xs0, w + int64_t(n_main) * ws0, ws0, y + n_main, ys0, M, tail, K, st);
  }
  if (use_big)
    return launch_tiled_cfg<256, 256, 2, 4, false, 2>(x, xs0, w, ws0, y, ys0, M, N, K,
                                                               st);
  const int64_t mid = int64_t((M + 127) / 128) * ((N + 127) / 128);
  if (mid < 2 * kCUs) {
    const int64_t narrow = int64_t((M + 127) / 128) * ((N + 63) / 64);
    if (narrow <= kCUs)
      return launch_tiled_cfg<128, 64, 2, 2, false, 4>(x, xs0, w, ws0, y, ys0, M, N,
                                                                K, st);
    return launch_tiled_cfg<128, 128, 2, 4, false, 4>(x, xs0, w, ws0, y, ys0, M, N, K,
                                                               st);
  }
  return launch_tiled_cfg<128, 128, 2, 2, false, 2>(x, xs0, w, ws0, y, ys0, M, N, K,
                                                             st);
}

struct SkinnyArgs {
  const bf16_t *x;
  int64_t xs0;
  const bf16_t *w;
  int64_t ws0;
  bf16_t *y;
  int64_t ys0;
  int M, N, K, split;
  float *part;
  int32_t *cnt;
  ProArgs pro;
};

template <int kNW, int kMT, int kNT, int kPro, int kEpi = 0>
void launch_skinny(const SkinnyArgs &a, hipStream_t st) {
  const int cols = 16 * (kEpi == 1 ? 1 : kNT);
  const dim3 grid(unsigned((a.N + cols - 1) / cols), unsigned(a.split));
  gemm_skinny_kernel<kNW, kMT, kNT, kPro, kEpi><<<grid, 64 * kNW, 0, st>>>(
      a.x, a.xs0, a.w, a.ws0, a.y, a.ys0, a.M, a.N, a.K, a.part, a.cnt, a.pro);
}

template <int kNW, int kNT, int kPro, int kEpi = 0>
void launch_skinny_m(const SkinnyArgs &a, hipStream_t st) {
  switch ((a.M + 15) / 16) {
    case 1: launch_skinny<kNW, 1, kNT, kPro, kEpi>(a, st); break;
    case 2: launch_skinny<kNW, 2, kNT, kPro, kEpi>(a, st); break;
    case 3: launch_skinny<kNW, 3, kNT, kPro, kEpi>(a, st); break;
    default: launch_skinny<kNW, 4, kNT, kPro, kEpi>(a, st); break;
  }
}

template <int kPro>
void launch_skinny_plan(const SkinnyArgs &a, int nt, int nw, hipStream_t st) {
  if (nt == 1) {
    if (nw == 4) launch_skinny_m<4, 1, kPro>(a, st);
    else if (nw == 8) launch_skinny_m<8, 1, kPro>(a, st);
    else launch_skinny_m<16, 1, kPro>(a, st);
  } else {
    if (nw == 4) launch_skinny_m<4, 2, kPro>(a, st);
    else if (nw == 8) launch_skinny_m<8, 2, kPro>(a, st);
    else launch_skinny_m<16, 2, kPro>(a, st);
  }
}

#ifndef WY_GEMM_SPLIT_MAX_BLOCKS
#define WY_GEMM_SPLIT_MAX_BLOCKS 128
#endif
#ifndef WY_GEMM_SPLIT_MIN_K
#define WY_GEMM_SPLIT_MIN_K 512
#endif

// Launch shape of the skinny kernel: columns per workgroup (16 * nt), K
// splits across workgroups, waves per workgroup.
struct SkinnyPlan {
  int nt, blocks, split, nw;
};
// Waves per workgroup for `groups` workgroups that each cover `ks` of K: grow
// from 4 while the grid holds fewer than 2048 waves, each wave keeps at least
// one 128-wide batch of k, and every wave's slice stays a multiple of 32
// (the kernel's tail loop steps 32 columns and must not cross into the next
// wave's slice).  ks is a multiple of 128, so 4 waves always divide it.
int skinny_waves(int groups, int ks) {
  int nw = 4;
  while (nw < 16 && groups * nw < 2048 && ks / (2 * nw) >= 128 && ks % (64 * nw) == 0) nw *= 2;
  return nw;
}

SkinnyPlan skinny_plan(int N, int K, bool gate_up_pairs = false) {
  SkinnyPlan p;
  // 32 columns per workgroup when N is large (each x load then feeds two
  // column tiles, halving the x bytes per column), else 16.  Gate/up pairs
  // (N output columns from 2N weight rows) always take two tiles, one of each
  // half: the same workgroups as the plain plan of 2N columns when 2N >= 4096.
  p.nt = gate_up_pairs || N >= 4096 ? 2 : 1;
  p.blocks = gate_up_pairs ? (N + 15) / 16 : (N + 16 * p.nt - 1) / (16 * p.nt);
  // Split K across workgroups until the grid covers the CUs once, keeping
  // at least WY_GEMM_SPLIT_MIN_K of K per workgroup.
  p.split = 1;
  while (p.blocks < WY_GEMM_SPLIT_MAX_BLOCKS && p.blocks * p.split < 256 &&
         K / (2 * p.split) >= WY_GEMM_SPLIT_MIN_K && (K / (2 * p.split)) % 128 == 0 &&
         p.split < kMaxSplit)
    p.split *= 2;
  // Waves: enough workgroups x waves to keep the CUs streaming, each wave at
  // least one 128-wide batch of k.
  p.nw = skinny_waves(p.blocks * p.split, K / p.split);
  return p;
}

}  // namespace

// Split-K workspace: kSplitCounters int32 counters (one per column block;
// zero before the first call, left zero by every call), then the fp32
// partial tiles [split][M][N] (contents irrelevant).
constexpr int kSplitCounters = 4096;
constexpr int64_t kSplitPartOffset = kSplitCounters * 4;

extern "C" int64_t wy_gemm_2d_workspace_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 128 || M > kSkinnyMaxM) return 0;
  const SkinnyPlan p = skinny_plan(N, K);
  if (p.split == 1 || p.blocks > kSplitCounters) return 0;
  return kSplitPartOffset + int64_t(p.split) * M * N * 4;
}

// Plan, pick the split-K workspace if one is given, and launch the skinny
// kernel with prologue `pro` (0 plain, 1 RMSNorm, 2 SwiGLU).
static int run_skinny(SkinnyArgs a, int pro, void *workspace, int64_t workspace_bytes,
                      hipStream_t st) {
  SkinnyPlan p = skinny_plan(a.N, a.K);
  const int64_t need = wy_gemm_2d_workspace_bytes(a.M, a.N, a.K);
  if (p.split > 1 && need > 0 && workspace_bytes >= need) {
    a.split = p.split;
    a.cnt = static_cast<int32_t *>(workspace);
    a.part = reinterpret_cast<float *>(static_cast<char *>(workspace) + kSplitPartOffset);
  } else if (p.split > 1) {  // no workspace: one workgroup per column block
    p.split = 1;
    p.nw = skinny_waves(p.blocks, a.K);
  }
  if (pro == 1) launch_skinny_plan<1>(a, p.nt, p.nw, st);
  else if (pro == 2) launch_skinny_plan<2>(a, p.nt, p.nw, st);
  else launch_skinny_plan<0>(a, p.nt, p.nw, st);
  return wyh::launch_status();
}

extern "C" int wy_gemm_2d(const void *x, const int64_t *x_strides, const void *w,
                          const int64_t *w_strides, void *y, const int64_t *y_strides, int M,
                          int N, int K, void *workspace, int64_t workspace_bytes,
                          void *stream) {
  if (!x || !x_strides || !w || !w_strides || !y || !y_strides) return WY_E_NULL;
  if (M < 0 || N < 0 || K <= 0 || K % 128) return WY_E_SHAPE;
  if (x_strides[1] != 1 || w_strides[1] != 1 || y_strides[1] != 1 || x_strides[0] % 8 ||
      w_strides[0] % 8 || x_strides[0] < K || w_strides[0] < K || y_strides[0] < N ||
      !wyh::aligned16(x) || !wyh::aligned16(w) || (reinterpret_cast<uintptr_t>(y) & 1u))
    return WY_E_LAYOUT;
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace) ||
      (reinterpret_cast<uintptr_t>(workspace) & 3u))
    return WY_E_LAYOUT;
  if (M == 0 || N == 0) return WY_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bf16_t *xb = static_cast<const bf16_t *>(x);
  const bf16_t *wb = static_cast<const bf16_t *>(w);
  bf16_t *yb = static_cast<bf16_t *>(y);
  if (M <= kSkinnyMaxM) {
    SkinnyArgs a{xb, x_strides[0], wb, w_strides[0], yb, y_strides[0], M, N, K, 1, nullptr,
                 nullptr, ProArgs{}};
    return run_skinny(a, 0, workspace, workspace_bytes, st);
  }
  // 32-bit buffer offsets within one 256-row band
  if (int64_t(256) * x_strides[0] * 2 >= INT32_MAX || int64_t(256) * w_strides[0] * 2 >= INT32_MAX)
    return WY_E_SHAPE;
  return launch_tiled(xb, x_strides[0], wb, w_strides[0], yb, y_strides[0], M, N, K, st);
}

extern "C" int wy_gemm_2d_rmsnorm(const void *x, int64_t x_stride0, const void *residual,
                                  int64_t residual_stride0, const void *norm_weight, float eps,
                                  void *x_out, int64_t x_out_stride0, const void *w,
                                  int64_t w_stride0, void *y, int64_t y_stride0, int M, int N,
                                  int K, void *workspace, int64_t workspace_bytes,
                                  void *stream) {
  if (!x || !norm_weight || !w || !y) return WY_E_NULL;
  if (M < 0 || N < 0 || K <= 0 || K % 256) return WY_E_SHAPE;
  if (M > kSkinnyMaxM) return WY_E_UNSUPPORTED;
  if (x_stride0 % 8 || w_stride0 % 8 || x_stride0 < K || w_stride0 < K || y_stride0 < N ||
      !wyh::aligned16(x) || !wyh::aligned16(w) || !wyh::aligned16(norm_weight) ||
      (reinterpret_cast<uintptr_t>(y) & 1u) ||
      (residual && (residual_stride0 % 8 || residual_stride0 < K || !wyh::aligned16(residual))) ||
      (x_out && (x_out_stride0 % 8 || x_out_stride0 < K || !wyh::aligned16(x_out))))
    return WY_E_LAYOUT;
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace) ||
      (reinterpret_cast<uintptr_t>(workspace) & 3u))
    return WY_E_LAYOUT;
  if (M == 0 || N == 0) return WY_OK;
  ProArgs pro{static_cast<const bf16_t *>(residual), residual_stride0,
              static_cast<const bf16_t *>(norm_weight), eps, static_cast<bf16_t *>(x_out),
              x_out_stride0, 0};
  SkinnyArgs a{static_cast<const bf16_t *>(x), x_stride0, static_cast<const bf16_t *>(w),
               w_stride0, static_cast<bf16_t *>(y), y_stride0, M, N, K, 1, nullptr, nullptr,
               pro};
  return run_skinny(a, 1, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int wy_gemm_2d_swiglu(const void *gate_up, int64_t gate_up_stride0, int64_t up_offset,
                                 const void *w, int64_t w_stride0, void *y, int64_t y_stride0,
                                 int M, int N, int K, void *workspace, int64_t workspace_bytes,
                                 void *stream) {
  if (!gate_up || !w || !y) return WY_E_NULL;
  if (M < 0 || N < 0 || K <= 0 || K % 128) return WY_E_SHAPE;
  if (M > kSkinnyMaxM) return WY_E_UNSUPPORTED;
  if (gate_up_stride0 % 8 || up_offset % 8 || up_offset < K || gate_up_stride0 < up_offset + K ||
      w_stride0 % 8 || w_stride0 < K || y_stride0 < N || !wyh::aligned16(gate_up) ||
      !wyh::aligned16(w) || (reinterpret_cast<uintptr_t>(y) & 1u))
    return WY_E_LAYOUT;
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace) ||
      (reinterpret_cast<uintptr_t>(workspace) & 3u))
    return WY_E_LAYOUT;
  if (M == 0 || N == 0) return WY_OK;
  ProArgs pro{nullptr, 0, nullptr, 0.f, nullptr, 0, up_offset};
  SkinnyArgs a{static_cast<const bf16_t *>(gate_up), gate_up_stride0,
               static_cast<const bf16_t *>(w), w_stride0, static_cast<bf16_t *>(y), y_stride0,
               M, N, K, 1, nullptr, nullptr, pro};
  return run_skinny(a, 2, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int64_t wy_gemm_2d_gate_up_swiglu_workspace_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 128 || M > kSkinnyMaxM) return 0;
  const SkinnyPlan p = skinny_plan(N, K, true);
  if (p.split == 1 || p.blocks > kSplitCounters) return 0;
  return kSplitPartOffset + int64_t(p.split) * M * 2 * N * 4;
}

extern "C" int wy_gemm_2d_gate_up_swiglu(const void *x, int64_t x_stride0, const void *w,
                                         int64_t w_stride0, void *y, int64_t y_stride0, int M,
                                         int N, int K, void *workspace, int64_t workspace_bytes,
                                         void *stream) {
  if (!x || !w || !y) return WY_E_NULL;
  if (M < 0 || N < 0 || K <= 0 || K % 128) return WY_E_SHAPE;
  if (M > kSkinnyMaxM && N % 128) return WY_E_UNSUPPORTED;
  if (x_stride0 % 8 || w_stride0 % 8 || x_stride0 < K || w_stride0 < K || y_stride0 < N ||
      !wyh::aligned16(x) || !wyh::aligned16(w) || (reinterpret_cast<uintptr_t>(y) & 1u))
    return WY_E_LAYOUT;
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace) ||
      (reinterpret_cast<uintptr_t>(workspace) & 3u))
    return WY_E_LAYOUT;
  if (M == 0 || N == 0) return WY_OK;
  if (M > kSkinnyMaxM) {
    // 256 x 256 tiles of 128 gate + 128 up columns; 32-bit buffer offsets
    if (int64_t(256) * x_stride0 * 2 >= INT32_MAX || int64_t(2) * N * w_stride0 * 2 >= INT32_MAX)
      return WY_E_SHAPE;
    return launch_tiled_cfg<256, 256, 2, 4, true, 2>(
        static_cast<const bf16_t *>(x), x_stride0, static_cast<const bf16_t *>(w), w_stride0,
        static_cast<bf16_t *>(y), y_stride0, M, N, K, static_cast<hipStream_t>(stream));
  }
  SkinnyArgs a{static_cast<const bf16_t *>(x), x_stride0, static_cast<const bf16_t *>(w),
               w_stride0, static_cast<bf16_t *>(y), y_stride0, M, N, K, 1, nullptr, nullptr,
               ProArgs{}};
  SkinnyPlan p = skinny_plan(N, K, true);
  const int64_t need = wy_gemm_2d_gate_up_swiglu_workspace_bytes(M, N, K);
  if (p.split > 1 && need > 0 && workspace_bytes >= need) {
    a.split = p.split;
    a.cnt = static_cast<int32_t *>(workspace);
    a.part = reinterpret_cast<float *>(static_cast<char *>(workspace) + kSplitPartOffset);
  } else if (p.split > 1) {
    p.split = 1;
    p.nw = skinny_waves(p.blocks, K);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (p.nw == 4) launch_skinny_m<4, 2, 0, 1>(a, st);
  else if (p.nw == 8) launch_skinny_m<8, 2, 0, 1>(a, st);
  else launch_skinny_m<16, 2, 0, 1>(a, st);
  return wyh::launch_status();
}
