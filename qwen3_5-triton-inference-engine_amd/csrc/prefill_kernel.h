// The varlen causal prefill kernel template, shared by prefill.hip (the
// queue-launch variants and the host side) and prefill_direct.hip (the
// one-workgroup-per-block variants, compiled with MFMA accumulators in
// VGPRs).
//
// Packed varlen causal GQA prefill attention on bf16 MFMA (gfx950).
//
// One launch; one workgroup = 4 wavefronts on (sequence b, KV head h,
// 32-token query block); wave w owns query head 4h + w, so the four heads of
// the GQA group share every K/V tile in LDS.
//
// Attention is computed transposed so that a lane owns one query row:
//   S^T = K Q^T      v_mfma_f32_32x32x16_bf16; A = K tile (LDS), B = q row
//                    (lane%32) kept in registers for the whole kernel.
//   O^T += V^T P^T   A = V^T, read from the row-major V tile in LDS with
//                    ds_read_b64_tr_b16 (the gfx950 transposing LDS read), B =
//                    P^T taken straight from the S^T accumulators.
// The K tile's LDS rows are a permutation of the 64 tokens, chosen so that
// the S^T accumulator registers of lane (col, g) hold tokens 32mt + 16g + r
// (r = register index 0..15): every PV k-step then needs 8 consecutive tokens
// of V, two transposing reads of 4 tokens each.  Row max / sum are lane-local
// plus one xor-32 exchange.  Softmax in base 2 with 1/sqrt(D) folded into
// log2(e); P is rounded to bf16 for PV as in the reference kernel
// (gqa_attention_varlen_causal.py:146-203).  The exponentials use a per-row
// reference fixed by the first KV tile instead of a running max, so O is
// never rescaled inside the loop (exact after the final 1/l); a row whose
// scores outgrow it by more than 2^64 sends the block through an exact
// two-pass recomputation.
//
// K and V tiles travel global -> LDS as buffer loads with the LDS-DMA bit (no
// registers), double-buffered: tile t+1 is in flight while tile t is
// consumed, one barrier per tile.  LDS rows are padded so the MFMA operand
// reads are conflict-free.  The DMAs are buffer loads whose range ends at the
// sequence's last row, so rows past the end are never fetched; their scores
// are masked to -inf, so their P is exactly 0.  Query blocks run heaviest
// first (LPT): as a grid of one workgroup per block when that grid fits the
// chip, otherwise as a persistent grid of one workgroup per CU drawing blocks
// from a shared ticket counter.
#pragma once

#include <atomic>
#include <type_traits>

#include "wy_common.h"

using namespace wy;

#if WY_TRACE
namespace {
__device__ unsigned long long g_trace[256 * 64 * 8];
}  // namespace
#endif

namespace wy_prefill {

constexpr int kD = 256;
constexpr int kG = 4;
constexpr int kBQ = 32;                  // query tokens per workgroup
constexpr int kBN = 64;                  // kv tokens per tile
// LDS rows are padded.  K rows are 32 + 1 16-byte slots (528 B): eight
// consecutive rows start on eight different 4-bank groups, so the b128 MFMA
// operand reads are conflict-free.  V rows are 32 + 4 slots (576 B): the four
// rows one half-wave reads per transposing load start 16 banks apart.
constexpr int kKSlots = kD / 8 + 1;      // 33 slots per K row
constexpr int kVSlots = kD / 8 + 4;      // 36 slots per V row
constexpr int kKPitch = kKSlots * 16;    // 528 B
constexpr int kQPitch = 528;             // q staging rows (512 B + 16 against bank conflicts)
constexpr int kVPitch = kVSlots * 16;    // 576 B
constexpr int kTileK = kBN * kKPitch;    // 33792 B
constexpr int kTileV = kBN * kVPitch;    // 36864 B
static_assert(2 * 32 * kQPitch <= kTileV, "two waves' q rows fit one V slot");
constexpr int kKDma = kTileK / 1024 + (kTileK % 1024 != 0);  // 1 KiB DMA blocks: 33
constexpr int kVDma = kTileV / 1024;                          // 36
static_assert(kTileV % 1024 == 0, "V tile is a whole number of DMA blocks");
constexpr int kRingBytes = 2 * (kTileK + kTileV);  // two K + two V slots: 138 KiB
// The K tile is 33 DMA blocks: in the steady tile loop every wave issues 9 K
// blocks, and the ninth of waves 1..3 lands in this unread 1 KiB, so the
// issue needs no branch.
constexpr int kLdsBytes = kRingBytes + 1024;
// Output staging in the epilogue (reuses the rings): 32 rows of 4 heads x
// 256 dims, rows padded by 16 bytes against bank conflicts of the lane writes.
constexpr int kStagePitch = 4 * 256 + 8;   // bf16
static_assert(32 * kStagePitch * 2 <= 2 * kTileV, "output stage fits the V ring");
// Exponentials are taken against a per-row reference fixed by the first KV
// tile; a later score may exceed it by a factor up to 2^64 (P stays finite in
// bf16 and fp32).  Beyond that the block is recomputed exactly.
// LDS of the queue launch's ticket -> block map: 2 n_seq + n_qblocks + 2 ints.
constexpr int kPlanLds = 4096;
constexpr float kHeadroomScale = 18446744073709551616.0f;  // 2^64

typedef __attribute__((address_space(3))) void lds_void_t;

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

__device__ __forceinline__ uint32_t lds_u32(const unsigned char *p) {
  return uint32_t(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) unsigned char *)(p)));
}

// ds_read_b64_tr_b16 (gfx950 transposing LDS read) as inline asm.  Issued
// through the builtin, the compiler waits for every in-flight LDS DMA before
// the read (it cannot tell the DMA targets from the tile being read), which
// would expose the DMA latency once per tile.  The caller waits for the data
// with lgkm_wait<N>(), which ties the destination registers so that nothing
// reads them earlier.  LDS reads complete in order, so lgkmcnt(N) with N the
// number of reads issued after the awaited ones is sufficient whatever other
// LDS or scalar-memory operations are interleaved.
template <int kOff>
__device__ __forceinline__ u32x2_t ds_read_tr16(uint32_t lds_addr) {
  u32x2_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(lds_addr), "i"(kOff));
  return r;
}
template <int kOff>
__device__ __forceinline__ u32x4_t ds_read_b128_at(uint32_t lds_addr) {
  u32x4_t r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(lds_addr), "i"(kOff));
  return r;
}
template <int kOff>
__device__ __forceinline__ void ds_write_b128_at(uint32_t lds_addr, const u32x4_t &v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(lds_addr), "v"(v), "i"(kOff) : "memory");
}
template <int kN>
__device__ __forceinline__ void lgkm_wait1(u32x4_t &a) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "n"(kN));
}
template <int kN>
__device__ __forceinline__ void lgkm_wait2(u32x2_t &a, u32x2_t &b) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "n"(kN));
}
template <int kN>
__device__ __forceinline__ void lgkm_wait(u32x2_t (&a)[4], u32x2_t (&b)[4]) {
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]),
                 "+v"(b[2]), "+v"(b[3])
               : "n"(kN));
}

// A row's values in lanes l and l + 32 (the two k-groups of the MFMA
// layouts): lo = the value of lane l % 32, hi = that of lane l % 32 + 32, in
// every lane, by one v_permlane32_swap (a VALU op; a shuffle through
// ds_bpermute waits in the LDS queue behind the operand reads and DMAs).
__device__ __forceinline__ void row_halves(float v, float &lo, float &hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}
__device__ __forceinline__ float row_max2(float v) {
  float lo, hi;
  row_halves(v, lo, hi);
  return fmaxf(lo, hi);
}
// lo + hi: the same sum, operand for operand, in both lanes of the row
__device__ __forceinline__ float row_sum2(float v) {
  float lo, hi;
  row_halves(v, lo, hi);
  return lo + hi;
}

// Token held by LDS row `row` of a K tile (see the header comment).
__device__ __forceinline__ int k_row_token(int row) {
  const int mt = row >> 5, r = row & 31;
  return 32 * mt + 16 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3);
}


// ------------------------------------------------------------------ attention
// Attention-block extras (kRot > 0): the raw q rows get the partial RoPE on
// dims [0, kRot) at their position ids, and the output is multiplied by
// sigmoid(gate) in the epilogue.
struct BlockArgs {
  const bf16_t *gate;  // [T, H_q, D] view, unit innermost stride
  int64_t gs_t, gs_h;
  const void *pos;     // position ids [T], int32 or int64
  int64_t ps_t;
  int pos64;
  const float *inv_freq;
  const float *rope_tab;  // [T][kRot]: sin of the kRot/2 angles, then cos
};

// One LDS DMA as inline asm: lane l's 16 bytes at buffer offset voff + soff
// land at LDS address m0 + 16 l.  The compiler does not see it, so it inserts
// no wait for it before its own LDS accesses; the kernel waits for it
// explicitly (s_waitcnt vmcnt) before any read of its target.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_lds_asm(__amdgpu_buffer_rsrc_t rs, uint32_t m0, uint32_t voff,
                                              uint32_t soff) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %3 offen lds"
               ::"v"(voff), "s"(rs), "s"(m0), "s"(soff)
               : "memory", "m0");
}
#pragma clang diagnostic pop
template <int kOff>
__device__ __forceinline__ void ds_write_b32_at(uint32_t addr, uint32_t v) {
  asm volatile("ds_write_b32 %0, %1 offset:%2" ::"v"(addr), "v"(v), "i"(kOff) : "memory");
}
template <int kOff>
__device__ __forceinline__ void ds_write_b64_at(uint32_t addr, u32x2_t v) {
  asm volatile("ds_write_b64 %0, %1 offset:%2" ::"v"(addr), "v"(v), "i"(kOff) : "memory");
}

template <bool kList, int kRot>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void varlen_causal_prefill_kernel(
    const bf16_t *__restrict__ q, int64_t qs_t, int64_t qs_h,
    const bf16_t *__restrict__ k, int64_t ks_t, int64_t ks_h,
    const bf16_t *__restrict__ v, int64_t vs_t, int64_t vs_h, bf16_t *__restrict__ out,
    int64_t os_t,
    int64_t os_h, const int32_t *__restrict__ cu, float qk_scale_log2, int n_seq,
    int n_kv_heads, int n_qblocks, int32_t *__restrict__ counters, const BlockArgs blk,
    int ticket_order) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_next_item;
  __shared__ __align__(16) uint32_t s_over[4];
  __shared__ int s_scan[256];
  __shared__ int plan_lds[kPlanLds];

  const int bh_count = n_seq * n_kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;     // k-group / row-quad selector of the MFMA layouts
  const int col = lane & 31;   // query row within the block

  // LDS: a two-slot ring of K tiles, then a two-slot ring of V tiles.  K
  // runs one tile ahead of V: iteration t computes S^T of tile t+1 (MFMA)
  // while the VALU turns S^T of tile t into P, then runs PV of tile t.
  unsigned char *const k_ring = smem;
  unsigned char *const v_ring = smem + 2 * kTileK;

  // Work distribution.  Direct launch (grid = every query block, used when
  // it fits the chip in one round): one block per workgroup, heaviest first
  // (LPT); workgroups are dealt to the 8 XCDs round-robin by id, so with
  // B * H_kv a multiple of 8 every query block of a (sequence, head) lands on
  // one XCD and its K/V re-reads hit that XCD's L2 (32 x 128 tokens: 17.7 -> 17.0
  // us against an order rotated across XCDs).  Queue launch (a persistent
  // grid of one workgroup per CU): the active query blocks, heaviest first,
  // are numbered by tickets drawn from a counter shared by all workgroups, so
  // a CU that finishes early takes the next block at once instead of waiting
  // for the in-order dispatcher, and inactive blocks cost nothing.  Each
  // workgroup derives the ticket -> block map itself (sequence lengths and
  // per-slice prefix counts in LDS); the next ticket is drawn late in each
  // block, after its last tile's barrier, and mapped in the epilogue.
  int item = int(blockIdx.x);
  int n_items = 0;
  int *const lens = plan_lds;               // [n_seq] sequence lengths
  int *const cu_l = plan_lds + n_seq;       // [n_seq + 1] cu_seqlens
  int *const pre = cu_l + n_seq + 1;        // [n_qblocks + 1] tickets before slice s
  if constexpr (kList) {
    for (int i = tid; i <= n_seq; i += 256) {
      const int c0 = cu[i];
      cu_l[i] = c0;
      if (i < n_seq) lens[i] = cu[i + 1] - c0;
    }
    __syncthreads();
    // pre[s + 1] = H_kv * #{b : len_b > 32 * qb(s)}, qb(s) = n_qblocks - 1 - s;
    // then an exclusive scan: each thread sums a contiguous run of slices,
    // the run totals are scanned, and the runs are rewritten as prefixes.
    const int per = (n_qblocks + 255) / 256;
    const int s_lo = min(tid * per, n_qblocks), s_hi = min(s_lo + per, n_qblocks);
    int run = 0;
    for (int sl = s_lo; sl < s_hi; ++sl) {
      const int thr = (n_qblocks - 1 - sl) * kBQ;
      int c = 0;
      for (int bb = 0; bb < n_seq; ++bb) c += lens[bb] > thr;
      pre[sl + 1] = c * n_kv_heads;
      run += c * n_kv_heads;
    }
    s_scan[tid] = run;
    __syncthreads();
    for (int o = 1; o < 256; o <<= 1) {
      const int x = tid >= o ? s_scan[tid - o] : 0;
      __syncthreads();
      s_scan[tid] += x;
      __syncthreads();
    }
    int acc = s_scan[tid] - run;
    for (int sl = s_lo; sl < s_hi; ++sl) {
      acc += pre[sl + 1];
      pre[sl + 1] = acc;
    }
    if (tid == 0) pre[0] = 0;
    __syncthreads();
    n_items = pre[n_qblocks];
    // The first ticket of workgroup i is i; the counter numbers the later
    // draws (ticket gridDim.x + counter), so no workgroup starts behind 255
    // others' atomics on one address.
  }
  // Test hook (wy_prefill_set_ticket_order): the same blocks in another
  // order.  0 heaviest first; 1 lightest first; 2 alternately from both ends.
  auto permute = [&](int it, int n) {
    if (ticket_order == 1) return n - 1 - it;
    if (ticket_order == 2) return (it & 1) ? n - 1 - (it >> 1) : (it >> 1);
    return it;
  };
#if WY_TRACE
  int trace_k = 0;
  unsigned long long tr0 = 0, tr1 = 0, tr2 = 0, trm = 0, trq = 0, tre = 0, trs = 0, tpf = 0, tsw = 0;
#endif
  // DMA one tile into a ring slot as wave-wide 1 KiB blocks (lane j fills
  // 16-byte slot 64*blk + j; pad slots get the row's first chunk, unread).
  // Wave w issues blocks w, w+4, ...  The DMAs are buffer loads over the
  // sequence's rows of this KV head: the per-lane row/chunk offsets are
  // tile-invariant registers computed once here, the tile offset is scalar,
  // and rows past the sequence's end fall outside the buffer's range (no
  // clamping arithmetic, nothing fetched).  Keeping the address registers
  // invariant also keeps the compiler from waiting on in-flight DMAs before
  // reusing them.
  constexpr int kKPerWave = (kKDma + 3) / 4;  // 9
  constexpr int kVPerWave = kVDma / 4;        // 9
  const uint32_t k_row_bytes = uint32_t(ks_t) * 2u;
  const uint32_t v_row_bytes = uint32_t(vs_t) * 2u;
  uint32_t k_voff[kKPerWave], v_voff[kVPerWave];
#pragma unroll
  for (int i = 0; i < kKPerWave; ++i) {
    const int sl = 64 * (wave + 4 * i) + lane;
    const int row = sl / kKSlots;
    const int c = sl - row * kKSlots;
    k_voff[i] = uint32_t(k_row_token(row < kBN ? row : kBN - 1)) * k_row_bytes +
                uint32_t(c < kD / 8 ? c : 0) * 16u;
  }
#pragma unroll
  for (int i = 0; i < kVPerWave; ++i) {
    const int sl = 64 * (wave + 4 * i) + lane;
    const int row = sl / kVSlots;
    const int c = sl - row * kVSlots;
    v_voff[i] = uint32_t(row) * v_row_bytes + uint32_t(c < kD / 8 ? c : 0) * 16u;
  }
  // Queue launch: ticket -> (sequence, KV head, query block).
  auto map_ticket = [&](int it, int &b_, int &h_, int &qb_) {
    const int tk = permute(it, n_items);
    // slice: the last s with pre[s] <= tk (64-ary search, one probe per lane)
    int lo = 0, hi = n_qblocks;
    while (hi - lo > 1) {
      const int step = (hi - lo + 63) / 64;
      const int probe = lo + lane * step;
      const bool le = probe < hi && pre[probe] <= tk;
      const int k = 63 - __builtin_clzll(__ballot(le));  // lane 0 always qualifies
      lo += k * step;
      hi = min(lo + step, hi);
    }
    qb_ = n_qblocks - 1 - lo;
    const int j = tk - pre[lo];
    const int pair = j / n_kv_heads;
    h_ = j - pair * n_kv_heads;
    // b: the pair-th sequence (ascending) longer than 32 * qb
    const int thr = qb_ * kBQ;
    int seen = 0;
    b_ = 0;
    for (int b0 = 0; b0 < n_seq; b0 += 64) {
      const uint64_t m = __ballot(b0 + lane < n_seq && lens[b0 + lane] > thr);
      const int c = __popcll(m);
      if (pair < seen + c) {
        // position of the (pair - seen)-th set bit of m
        const bool mine = ((m >> lane) & 1) &&
                          __popcll(m & ((uint64_t(1) << lane) - 1)) == pair - seen;
        b_ = b0 + (__builtin_ctzll(__ballot(mine)));
        break;
      }
      seen += c;
    }
  };
  // Block coordinates.  In the queue launch a block maps the next ticket and
  // requests that block's q rows and first tiles before its own output
  // stores (`pf`): the memory counter completes in order, so requested after
  // the stores they would wait for them.
  int b = 0, h = 0, qb = 0;
  bool pf = false;
  u32x4_t xr_pf[16];
  // q rows of a block in the row layout: buffer loads over a range that ends
  // after the sequence's last row, so rows past it read zeros; the row step
  // is the scalar offset, the lane's place in a row pair the only vector
  // offset (per-row clamped addresses were hoisted out of the block loop by
  // the compiler and spilled).
  auto load_q_rows = [&](int start_, int n_, int q0_, int h_) {
    const uint32_t row_b = uint32_t(qs_t) * 2u;
    const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16_t *>(q + (int64_t(start_) + q0_) * qs_t + (h_ * kG + wave) * qs_h), 0,
        int(uint32_t(n_ - 1 - q0_) * row_b + kD * 2), 0x00020000);
    const uint32_t vo = uint32_t(lane >> 5) * row_b + uint32_t(lane & 31) * 16u;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      xr_pf[i] = __builtin_amdgcn_raw_buffer_load_b128(qr, vo, uint32_t(2 * i) * row_b, 0);
  };
  auto mk_rsrc = [&](const bf16_t *base, int64_t st_t, int64_t st_h, int start_, int n_, int h_,
                     uint32_t row_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16_t *>(base + int64_t(start_) * st_t + h_ * st_h), 0,
        int(uint32_t(n_ - 1) * row_bytes + kD * 2), 0x00020000);
  };
  auto dma_k = [&](__amdgpu_buffer_rsrc_t rs, int t, int slot, int i0, int i1) {
    const uint32_t soff = uint32_t(t * kBN) * k_row_bytes;
#pragma unroll
    for (int i = i0; i < i1; ++i) {
      if (wave + 4 * i < kKDma)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (lds_void_t *)(k_ring + slot * kTileK + (wave + 4 * i) * 1024), 16, k_voff[i],
            soff, 0, 0);
    }
  };
  auto dma_v = [&](__amdgpu_buffer_rsrc_t rs, int t, int slot, int i0, int i1) {
    const uint32_t soff = uint32_t(t * kBN) * v_row_bytes;
#pragma unroll
    for (int i = i0; i < i1; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (lds_void_t *)(v_ring + slot * kTileV + (wave + 4 * i) * 1024), 16, v_voff[i],
          soff, 0, 0);
  };
  // the next ticket: every thread issues the atomic, only thread 0's offset
  // lies inside the 4-byte range (a branch around it would make the merge of
  // its result wait for every memory operation in flight)
  const __amdgpu_buffer_rsrc_t ticket_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(counters, 0, 4, 0x00020000);
  for (;;) {
#if WY_TRACE
  tr0 = __builtin_amdgcn_s_memrealtime();
#endif
  if constexpr (kList) {
    if (item >= n_items) {  // uniform: the queue is drained
      // The last workgroup to get here leaves both counters at zero for the
      // next launch (every workgroup has drawn its final ticket by then).
      if (tid == 0 && atomicAdd(&counters[1], 1) == int(gridDim.x) - 1) {
        __hip_atomic_store(&counters[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&counters[1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      return;
    }
    if (!pf) map_ticket(item, b, h, qb);
  } else {
    const int it = permute(item, int(gridDim.x));
    const int slice = it / bh_count;
    const int bh = it - slice * bh_count;
    b = bh / n_kv_heads;
    h = bh - b * n_kv_heads;
    qb = n_qblocks - 1 - slice;
  }
  const int start = kList ? cu_l[b] : cu[b];
  const int n = kList ? lens[b] : cu[b + 1] - start;
  const int q0 = qb * kBQ;
  if (q0 >= n) return;  // direct launch only (the queue holds active blocks only)

  const int qrow = q0 + col;

  const int kv_end = min(q0 + kBQ, n);  // exclusive bound of keys any row can see
  const int n_tiles = (kv_end + kBN - 1) / kBN;

  const __amdgpu_buffer_rsrc_t k_rsrc = mk_rsrc(k, ks_t, ks_h, start, n, h, k_row_bytes);
  const __amdgpu_buffer_rsrc_t v_rsrc = mk_rsrc(v, vs_t, vs_h, start, n, h, v_row_bytes);
  // Issue K (V) blocks [i0, i1) of this wave for tile t into `slot`.
  auto issue_k = [&](int t, int slot, int i0, int i1) { dma_k(k_rsrc, t, slot, i0, i1); };
  auto issue_v = [&](int t, int slot, int i0, int i1) { dma_v(v_rsrc, t, slot, i0, i1); };
  auto issue_first = [&] {
    issue_k(0, 0, 0, kKPerWave);
    issue_v(0, 0, 0, kVPerWave);
    if (n_tiles > 1) issue_k(1, 1, 0, kKPerWave);
  };

  // V rows past the sequence's end are not fetched; their P is 0, so their
  // LDS rows only need to hold finite values: zero the V ring once when the
  // last tile is partial.
  if (!pf && n < n_tiles * kBN) {
    for (int o = tid * 16; o < 2 * kTileV; o += 256 * 16)
      st16(v_ring + o, u32x4_t{0u, 0u, 0u, 0u});
    __syncthreads();
  }
  // q row as the B operand of S^T, one 16-byte slice per 16-dim k-step,
  // pre-multiplied by scale*log2(e) and rounded to bf16 as the reference does
  // (gqa_attention_varlen_causal.py:146,158): scores come out in log2 units.
  // The q loads are issued before the first tiles' DMA, so they do not queue
  // behind it; the conversion waits for q only.  Each wave loads its head's
  // 32 rows whole (two 512-byte rows per load instruction) and regroups them
  // through LDS into the lanes' 16-byte slices: the V slot of tile 1, not
  // written before the first tile loop, holds two waves' rows at a time.
#if WY_TRACE
  trm = __builtin_amdgcn_s_memrealtime();
#endif
  bf16x8_t qb_op[16];
  // Attention block: the gate values of the pieces this thread stores in the
  // epilogue (rows r0, r0 + 2, ..., 16 bytes at column c8 of the 4 heads'
  // 2 KiB row), whole rows per load instruction.  Requested after the
  // block's last QK, when the q operand's registers are free, so that the
  // 64 registers they take are not held through the tile loop, and the last
  // tile's softmax and PV hide their latency.
  static_assert(kG * kD == 1024, "two output rows per workgroup step");
  const int r0 = tid >> 7, c8 = (tid & 127) * 8;
  u32x4_t gate_c[kRot > 0 ? kBQ / 2 : 1];
  auto load_gate = [&] {
    if constexpr (kRot > 0) {
      // (the range ends after the last row's fourth head: every byte in it
      // lies inside the gate tensor; rows past the sequence are not stored)
      const uint32_t row_b = uint32_t(blk.gs_t) * 2u, head_b = uint32_t(blk.gs_h) * 2u;
      const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<bf16_t *>(blk.gate + (int64_t(start) + q0) * blk.gs_t + (h * kG) * blk.gs_h),
          0, int(uint32_t(n - 1 - q0) * row_b + (kG - 1) * head_b + kD * 2), 0x00020000);
      const uint32_t vo = uint32_t(r0) * row_b + uint32_t(c8 / kD) * head_b + uint32_t(c8 % kD) * 2u;
#pragma unroll
      for (int i = 0; i < kBQ / 2; ++i)
        gate_c[i] = __builtin_amdgcn_raw_buffer_load_b128(gr, vo, uint32_t(2 * i) * row_b, 0);
    }
  };
  {
    // (a prefetched block's rows were requested by the previous epilogue)
    if (!pf) load_q_rows(start, n, q0, h);
    u32x4_t(&xr)[16] = xr_pf;
    f32x4_t tsn[kRot > 0 ? kRot / 16 : 1], tcs[kRot > 0 ? kRot / 16 : 1];
    if constexpr (kRot > 0) {
      const int qc = qrow < n ? qrow : n - 1;
      const float *tr = blk.rope_tab + (int64_t(start) + qc) * kRot + 8 * g;
#pragma unroll
      for (int kk = 0; kk < kRot / 32; ++kk)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          tsn[2 * kk + u] = *reinterpret_cast<const f32x4_t *>(tr + 16 * kk + 4 * u);
          tcs[2 * kk + u] = *reinterpret_cast<const f32x4_t *>(tr + kRot / 2 + 16 * kk + 4 * u);
        }
    }
    if (!pf) issue_first();
    {
      // LDS accesses as inline asm: a prefetched block's DMAs may be in
      // flight, and the compiler would make compiler-visible accesses wait
      // for them.
      const uint32_t qst = lds_u32(v_ring + kTileV + (wave & 1) * (kBQ * kQPitch));
      const uint32_t qw = qst + uint32_t((lane >> 5) * kQPitch + (lane & 31) * 16);
      const uint32_t qr = qst + uint32_t(col * kQPitch + g * 16);
#pragma unroll
      for (int round = 0; round < 2; ++round) {
        if ((wave >> 1) == round) {
          static_for<0, 16>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            ds_write_b128_at<2 * i * kQPitch>(qw, xr[i]);
          });
          static_for<0, 16>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            xr[i] = ds_read_b128_at<i * 32>(qr);
          });
          asm volatile("s_waitcnt lgkmcnt(0)"
                       : "+v"(xr[0]), "+v"(xr[1]), "+v"(xr[2]), "+v"(xr[3]), "+v"(xr[4]),
                         "+v"(xr[5]), "+v"(xr[6]), "+v"(xr[7]), "+v"(xr[8]), "+v"(xr[9]),
                         "+v"(xr[10]), "+v"(xr[11]), "+v"(xr[12]), "+v"(xr[13]), "+v"(xr[14]),
                         "+v"(xr[15])::"memory");
          if (round == 1 && n < n_tiles * kBN) {
            // the slot must hold finite values past the sequence (see above)
            const u32x4_t z = {0u, 0u, 0u, 0u};
            static_for<0, 16>([&](auto ic) {
              constexpr int i = decltype(ic)::value;
              ds_write_b128_at<2 * i * kQPitch>(qw, z);
            });
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          }
        }
        if (round == 0) __syncthreads();
      }
    }
    if constexpr (kRot > 0) {
      // Partial RoPE of the raw row, the standalone kernel's device math and
      // bf16 rounding (partial_rope.py:74-98): k-step kk < kRot/32 holds dims
      // 16kk + 8g .. +7 of the first half, k-step kk + kRot/32 their partners.
      // sin / cos come from the K/V launch's table (the same rope_sincos
      // values the standalone kernel computes).
      static_assert(kRot % 32 == 0 && kRot <= kD, "rotary dims in whole k-step pairs");
      constexpr int kH = kRot / 32;
#pragma unroll
      for (int kk = 0; kk < kH; ++kk) {
        u32x4_t a = xr[kk], bb = xr[kk + kH];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const f32x4_t &sv = tsn[2 * kk + w / 2], &cv = tcs[2 * kk + w / 2];
          const float s0 = sv[2 * (w & 1)], s1 = sv[2 * (w & 1) + 1];
          const float c0 = cv[2 * (w & 1)], c1 = cv[2 * (w & 1) + 1];
          float o1l, o2l, o1h, o2h;
          rope_rotate(bf16_lo(a[w]), bf16_lo(bb[w]), c0, s0, o1l, o2l);
          rope_rotate(bf16_hi(a[w]), bf16_hi(bb[w]), c1, s1, o1h, o2h);
          a[w] = pack_bf16x2(o1l, o1h);
          bb[w] = pack_bf16x2(o2l, o2h);
        }
        xr[kk] = a;
        xr[kk + kH] = bb;
      }
    }
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      u32x4_t x = xr[kk];
      if (qrow >= n) x = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
      for (int w = 0; w < 4; ++w)
        x[w] = pack_bf16x2(bf16_lo(x[w]) * qk_scale_log2, bf16_hi(x[w]) * qk_scale_log2);
      qb_op[kk] = __builtin_bit_cast(bf16x8_t, x);
    }
  }

#if WY_TRACE
  trq = __builtin_amdgcn_s_memrealtime();
#endif
  // S^T of the tile in K slot `slot`: register r of slab mt = token 32mt+16g+r.
  // dma(kb) is called after k-step block kb so the next tiles' DMA issue is
  // spread between the MFMAs instead of stalling the wave in one burst.
  // The accumulators start at `init` (0, or -m_ref once the row reference is
  // known, so the MFMAs deliver s - m_ref directly).
  auto qk = [&](int slot, f32x16_t(&sc)[2], const f32x16_t &init, auto &&dma) {
    sc[0] = init;
    sc[1] = init;
    const unsigned char *kr = k_ring + slot * kTileK + col * kKPitch + g * 16;
    u32x4_t ka[2][8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ka[0][i] = ld16(kr + (i & 1) * 32 * kKPitch + (i >> 1) * 32);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int cur = kb & 1;
      if (kb + 1 < 4) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          ka[cur ^ 1][i] = ld16(kr + (i & 1) * 32 * kKPitch + (4 * (kb + 1) + (i >> 1)) * 32);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        sc[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, ka[cur][i]), qb_op[4 * kb + (i >> 1)], sc[i & 1], 0,
            0, 0);
      dma(kb);
    }
  };
  auto no_dma = [](int) {};
  f32x16_t zero16;
#pragma unroll
  for (int e = 0; e < 16; ++e) zero16[e] = 0.f;

  f32x16_t o[8];
  float l_part = 0.f;
  float m_ref = 0.f;  // per-row reference max (log2 units) of the exponentials
  const int row_lim = min(qrow, n - 1);  // last key this row may attend to
  const int l16 = lane & 15;
  const uint32_t v_lane_off =
      uint32_t((16 * g + (l16 >> 2)) * kVPitch + (16 * ((lane >> 4) & 1) + 4 * (l16 & 3)) * 2);

  // One pass over the KV tiles.  kMode 0: m_ref = row max of the first tile
  // (it always holds the row's first token); later tiles accumulate against
  // it.  A later score may exceed it; if one does by more than a factor 2^64,
  // the row sum l exceeds 2^64 and the caller redoes the block.
  // kMode 1: exact row max only (no PV).  kMode 2: accumulate against the
  // exact m_ref of a preceding kMode-1 pass.  There is no rescaling of O
  // inside the loop.  Once m_ref is known, S^T tiles are computed with their
  // accumulators started at -m_ref (tile 0 and 1 of kMode 0 subtract on the
  // VALU), and only tiles that reach the diagonal are masked.
  auto run_pass = [&](auto mode) {
    constexpr int kMode = decltype(mode)::value;
    float m_acc = -INFINITY;
    f32x16_t neg_m;
#pragma unroll
    for (int e = 0; e < 16; ++e) neg_m[e] = -m_ref;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    f32x16_t s_cur[2];
    qk(0, s_cur, kMode == 2 ? neg_m : zero16, no_dma);
    for (int t = 0; t < n_tiles; ++t) {
      const int kv0 = t * kBN;
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // K(t+1), V(t) landed
      __syncthreads();  // and every wave is done with S^T(t) and PV(t-1)
      const bool k_next = t + 2 < n_tiles, v_next = t + 1 < n_tiles;  // uniform
      // s_cur holds s - m_ref (biased) or s
      const bool biased = kMode == 2 || (kMode == 0 && t >= 2);

      // S^T of tile t+1 (none after the last tile), with the DMA of K(t+2)
      // and V(t+1) issued between its k-steps.
      f32x16_t s_nxt[2];
      if (v_next) {
        qk((t + 1) & 1, s_nxt, (kMode == 2 || (kMode == 0 && t >= 1)) ? neg_m : zero16,
           [&](int kb) {
             if (kb == 0 && k_next) issue_k(t + 2, t & 1, 0, 5);
             if (kb == 1 && k_next) issue_k(t + 2, t & 1, 5, kKPerWave);
             if (kb == 2) issue_v(t + 1, (t + 1) & 1, 0, 5);
             if (kb == 3) issue_v(t + 1, (t + 1) & 1, 5, kVPerWave);
           });
      }

      // ---- P of tile t (VALU; overlaps the MFMAs above) -------------------
      if (kv0 + kBN - 1 > q0) {  // the tile reaches the diagonal: mask
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const int thr = row_lim - (kv0 + 32 * mt + 16 * g);  // keep registers e <= thr
#pragma unroll
          for (int e = 0; e < 16; ++e) s_cur[mt][e] = e > thr ? -INFINITY : s_cur[mt][e];
        }
      }
      if (kMode == 1 || (kMode == 0 && t == 0)) {
        float mx = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s_cur[mt][e]);
        mx = row_max2(mx);
        if constexpr (kMode == 1) m_acc = fmaxf(m_acc, mx);
        else {
          m_ref = mx;
#pragma unroll
          for (int e = 0; e < 16; ++e) neg_m[e] = -mx;
        }
      }
      if constexpr (kMode != 1) {
        const float sub = biased ? 0.f : m_ref;
        float psum = 0.f;
        u32x4_t pb[4];  // P^T B operands: k-step 2mt+kk = tokens 32mt+16g+8kk .. +7
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const float a = __builtin_amdgcn_exp2f(s_cur[mt][8 * kk + 2 * w] - sub);
              const float c = __builtin_amdgcn_exp2f(s_cur[mt][8 * kk + 2 * w + 1] - sub);
              psum += a + c;
              pb[2 * mt + kk][w] = pack_bf16x2(a, c);
            }
        l_part += psum;

        // ---- O^T += V^T P^T of tile t ---------------------------------------
        // A operand of k-step ks = (mt, kk), dim block dt: lane (m = lane%32,
        // g) needs V[32mt + 16g + 8kk + 0..7][32dt + m].  A transposing read
        // hands lane i of each 16-lane group element i%4 of the 8-byte chunks
        // addressed by lanes 4j + i/4 (j = 0..3), so lane L addresses token
        // row 16g + L%16/4 (+4 for the second half) at dims 32dt + 16(L/16%2)
        // + 4(L%4).
        const uint32_t vr = lds_u32(v_ring + (t & 1) * kTileV) + v_lane_off;
        u32x2_t vlo[2][4], vhi[2][4];
        auto vload = [&](auto dtc, auto bufc) {
          constexpr int dt = decltype(dtc)::value, buf = decltype(bufc)::value;
          static_for<0, 4>([&](auto ksc) {
            constexpr int ks = decltype(ksc)::value;
            constexpr int off = (32 * (ks >> 1) + 8 * (ks & 1)) * kVPitch + dt * 64;
            vlo[buf][ks] = ds_read_tr16<off>(vr);
            vhi[buf][ks] = ds_read_tr16<off + 4 * kVPitch>(vr);
          });
        };
        vload(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
        static_for<0, 8>([&](auto dtc) {
          constexpr int dt = decltype(dtc)::value, cur = dt & 1;
          if constexpr (dt + 1 < 8) {
            vload(std::integral_constant<int, dt + 1>{}, std::integral_constant<int, cur ^ 1>{});
            lgkm_wait<8>(vlo[cur], vhi[cur]);  // this block's 8 reads have landed
          } else {
            lgkm_wait<0>(vlo[cur], vhi[cur]);
          }
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const u32x4_t a = {vlo[cur][ks][0], vlo[cur][ks][1], vhi[cur][ks][0], vhi[cur][ks][1]};
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                            __builtin_bit_cast(bf16x8_t, pb[ks]),
                                                            o[dt], 0, 0, 0);
          }
        });
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) s_cur[mt] = s_nxt[mt];
    }
    if constexpr (kMode == 1) m_ref = m_acc;
  };


  // The pass the kernel normally takes (the first-tile reference of kMode 0
  // above, same arithmetic), as a software pipeline with no branch inside a
  // tile: after the barrier of tile t the wave issues S^T(t+1) on the MFMA
  // pipe and, between those MFMAs, turns S^T(t) into P (exponentials, row
  // sum, bf16 packing) and issues the next tiles' DMA, so the VALU work runs
  // under the MFMAs instead of after them; then PV(t), its V operands
  // streamed a window of 8 MFMAs ahead, with the score registers handed on
  // for the next tile in its gaps.  Every LDS operand read is inline asm
  // with an explicit lgkmcnt count (LDS reads complete in order).  In the
  // last loop iteration the K DMA of the tile past the end lies outside the
  // buffer range (nothing fetched) and lands in a slot nobody reads again.
  // Only the last tile reaches the diagonal or the sequence end, so only it
  // is masked, after the loop.
  const uint32_t k_lane = lds_u32(k_ring) + uint32_t(col * kKPitch + g * 16);
  auto issue_k1 = [&](int t, int slot, auto ic) {
    constexpr int i = decltype(ic)::value;
    const uint32_t soff = uint32_t(t * kBN) * k_row_bytes;
    unsigned char *dst = k_ring + slot * kTileK + (wave + 4 * i) * 1024;
    if constexpr (4 * i + 3 >= kKDma) dst = wave + 4 * i < kKDma ? dst : smem + kRingBytes;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(k_rsrc, (lds_void_t *)dst, 16, k_voff[i], soff, 0,
                                             0);
  };
  auto issue_v1 = [&](int t, int slot, auto ic) {
    constexpr int i = decltype(ic)::value;
    const uint32_t soff = uint32_t(t * kBN) * v_row_bytes;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        v_rsrc, (lds_void_t *)(v_ring + slot * kTileV + (wave + 4 * i) * 1024), 16, v_voff[i],
        soff, 0, 0);
  };
  // Operand of S^T MFMA i (i = 8 kb + 2 c + mt): K rows 32 mt + col, k-step
  // 4 kb + c; of PV MFMA j (j = 8 ks + dt): V^T of dims 32 dt.., k-step ks.
  auto k_read = [&](uint32_t base, auto ic) {
    constexpr int i = decltype(ic)::value;
    constexpr int off = (i & 1) * 32 * kKPitch + (4 * (i >> 3) + ((i & 7) >> 1)) * 32;
    return ds_read_b128_at<off>(base);
  };
  auto v_read = [&](uint32_t base, u32x2_t &lo, u32x2_t &hi, auto jc) {
    constexpr int j = decltype(jc)::value;
    constexpr int ks = j >> 3, dt = j & 7;
    constexpr int off = (32 * (ks >> 1) + 8 * (ks & 1)) * kVPitch + dt * 64;
    lo = ds_read_tr16<off>(base);
    hi = ds_read_tr16<off + 4 * kVPitch>(base);
  };
  auto softmax_pair = [&](f32x16_t(&s)[2], u32x4_t(&pb)[4], float &psum, auto pc) {
    constexpr int p = decltype(pc)::value;
    constexpr int mt = p >> 3, kk = (p >> 2) & 1, w = p & 3;
    const float a = __builtin_amdgcn_exp2f(s[mt][8 * kk + 2 * w]);
    const float c = __builtin_amdgcn_exp2f(s[mt][8 * kk + 2 * w + 1]);
    psum += a + c;
    pb[2 * mt + kk][w] = pack_bf16x2(a, c);
  };
  auto mask_tile = [&](f32x16_t(&s)[2], int t) {
    const int kv0 = t * kBN;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int thr = row_lim - (kv0 + 32 * mt + 16 * g);  // keep registers e <= thr
#pragma unroll
      for (int e = 0; e < 16; ++e) s[mt][e] = e > thr ? -INFINITY : s[mt][e];
    }
  };
  // O^T += V^T P^T of the tile in V slot `vslot`; `gap(j)` runs after MFMA j.
  auto pv = [&](int vslot, u32x4_t(&pb)[4], auto &&gap) {
    const uint32_t vr = lds_u32(v_ring + vslot * kTileV) + v_lane_off;
    u32x2_t va[8][2];
    static_for<0, 8>([&](auto jc) { v_read(vr, va[jc][0], va[jc][1], jc); });
    static_for<0, 32>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      constexpr int ks = j >> 3, dt = j & 7, rest = 31 - j < 7 ? 31 - j : 7;
      lgkm_wait2<2 * rest>(va[j & 7][0], va[j & 7][1]);
      const u32x4_t a = {va[j & 7][0][0], va[j & 7][0][1], va[j & 7][1][0], va[j & 7][1][1]};
      o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                      __builtin_bit_cast(bf16x8_t, pb[ks]),
                                                      o[dt], 0, 0, 0);
      if constexpr (j + 8 < 32) v_read(vr, va[j & 7][0], va[j & 7][1], std::integral_constant<int, j + 8>{});
      gap(jc);
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  int nitem = 0, nb = 0, nh = 0, nqb = 0, nn = 0, nstart = 0, ntiles = 0;
  bool npf = false;
  auto prefetch_q = [&] {
    nitem = s_next_item;
    if (nitem < n_items) {  // uniform
      map_ticket(nitem, nb, nh, nqb);
      nstart = cu_l[nb];
      nn = lens[nb];
      ntiles = (min(nqb * kBQ + kBQ, nn) + kBN - 1) / kBN;
      load_q_rows(nstart, nn, nqb * kBQ, nh);
      npf = true;
    } else {
      // (defined on both paths: otherwise this block's q rows would stay
      // live through its whole tile loop for the path without a next block)
#pragma unroll
      for (int i = 0; i < 16; ++i) xr_pf[i] = u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  // Plain queue launch (kEarly): the next block's coordinates, q rows and K
  // tiles 0 and 1 are requested right after the barrier of this block's
  // last tile -- the K ring is free once every wave has computed the last
  // S^T -- so that their latency hides behind the last tile's softmax and PV
  // and the epilogue.  Its K DMAs are inline asm, and every LDS access after
  // them is too (the exact-fallback vote, the staging): the compiler would
  // make a visible LDS access wait for a DMA it knows of, and with it, by
  // the in-order memory counter, for the q rows.
  constexpr bool kEarly = kList && kRot == 0;
  auto prefetch_k = [&] {
    if (npf) {
      const __amdgpu_buffer_rsrc_t nk = mk_rsrc(k, ks_t, ks_h, nstart, nn, nh, k_row_bytes);
#pragma unroll
      for (int slot = 0; slot < 2; ++slot) {
        if (slot == 1 && ntiles < 2) break;
        const uint32_t soff = uint32_t(slot * kBN) * k_row_bytes;
#pragma unroll
        for (int i = 0; i < kKPerWave; ++i)
          dma16_lds_asm(nk,
                        wave + 4 * i < kKDma
                            ? lds_u32(k_ring + slot * kTileK + (wave + 4 * i) * 1024)
                            : lds_u32(smem + kRingBytes),
                        k_voff[i], soff);
      }
    }
  };
  // Queue launch: the next ticket is drawn late in the block -- at the top
  // of its last loop iteration (kEarly) or after the barrier of its last
  // tile, right after the first wait in a one-tile block -- early enough to
  // map it and prefetch that block, late enough that the last tickets of the
  // queue go to workgroups about to need them (drawn at the start of a long
  // block, a light ticket waited for the whole block while other workgroups
  // found the queue empty).
  int next_ticket = 0;
  auto draw_ticket = [&] {
    if constexpr (kList)
      next_ticket = __builtin_amdgcn_raw_ptr_buffer_atomic_add_i32(1, ticket_rsrc, tid * 4, 0, 0);
  };
  auto run_fast = [&] {
    // q, K(0), K(1) landed (and V(0), unless prefetched).  A prefetched
    // block's q rows and K tiles were requested before the previous block's
    // V(0) DMA and 16 output stores; younger than them are that DMA, the
    // stores and (attention block) the sin / cos loads, which may still be
    // in flight: V(0) is first read by PV(0), after the loop-top wait of
    // tile 0, or in a one-tile block after the wait below.
    if (pf)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(16 + kVPerWave + (kRot > 0 ? kRot / 8 : 0))
                   : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (n_tiles == 1) draw_ticket();
    f32x16_t s_cur[2], s_nxt[2];
#if WY_TRACE
    tr1 = __builtin_amdgcn_s_memrealtime();
#endif
    qk(0, s_cur, zero16, no_dma);
    if (n_tiles == 1) mask_tile(s_cur, 0);
    {
      float mx = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s_cur[mt][e]);
      m_ref = row_max2(mx);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e) s_cur[mt][e] -= m_ref;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e) s_nxt[mt][e] = -m_ref;
    }
    int t = 0;
    for (; t + 1 < n_tiles; ++t) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // K(t+1), V(t) landed
      __syncthreads();  // and every wave is done with S^T(t) and PV(t-1)
      if constexpr (kEarly) {
        if (t + 2 == n_tiles) draw_ticket();  // a tile ahead of its use
      }
      const uint32_t kb = k_lane + uint32_t(((t + 1) & 1) * kTileK);
      constexpr int kKW = 8;  // K operands in flight (MFMAs ahead)
      u32x4_t ka[kKW];
      static_for<0, kKW>([&](auto ic) { ka[ic] = k_read(kb, ic); });
      u32x4_t pb[4];
      float psum = 0.f;
      const uint32_t vr0 = lds_u32(v_ring + (t & 1) * kTileV) + v_lane_off;
      static_for<0, 32>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        constexpr int ii = i & 7, mt = ii & 1, ks = 4 * (i >> 3) + (ii >> 1);
        constexpr int wi = i % kKW;
        lgkm_wait1<(i + kKW <= 32 ? kKW - 1 : 31 - i)>(ka[wi]);
        s_nxt[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, ka[wi]), qb_op[ks], s_nxt[mt], 0, 0, 0);
        if constexpr (i + kKW < 32) ka[wi] = k_read(kb, std::integral_constant<int, i + kKW>{});
        // one P pair per odd MFMA; the next tiles' DMA (K(t+2), then V(t+1))
        // one block per MFMA
        if constexpr (i & 1) softmax_pair(s_cur, pb, psum, std::integral_constant<int, i / 2>{});
        if constexpr (i < 9) issue_k1(t + 2, t & 1, ic);
        else if constexpr (i < 18) issue_v1(t + 1, (t + 1) & 1, std::integral_constant<int, i - 9>{});
        __builtin_amdgcn_sched_barrier(0);
      });
      (void)vr0;
      l_part += psum;
      pv(t & 1, pb, [&](auto jc) {
        constexpr int j = decltype(jc)::value;
        constexpr int mt = j >> 4, e = j & 15;
        s_cur[mt][e] = s_nxt[mt][e];
        s_nxt[mt][e] = -m_ref;
      });
    }
    if (n_tiles > 1) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // V(t) landed
      __syncthreads();
      if constexpr (!kEarly) draw_ticket();
      mask_tile(s_cur, t);
    }
    // A prefetched one-tile block: its V(0) (every wave's part) has landed
    // before PV(0) reads it; with kEarly the barrier below serves.
    if (pf && n_tiles == 1) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if constexpr (!kEarly) asm volatile("s_barrier" ::: "memory");
    }
    if constexpr (kEarly) {
      // every wave is past its last S^T (the barrier above, or this one in
      // a one-tile block) before the next block's K tiles land
      if (tid == 0) s_next_item = next_ticket + int(gridDim.x);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      prefetch_q();
      prefetch_k();
    }
    load_gate();
    u32x4_t pb[4];
    float psum = 0.f;
    static_for<0, 16>([&](auto pc) { softmax_pair(s_cur, pb, psum, pc); });
    l_part += psum;
    pv(t & 1, pb, [](auto) {});
  };

  auto zero_acc = [&] {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
    l_part = 0.f;
  };

  zero_acc();
  run_fast();
  // (published to the workgroup through s_next_item before the barrier below)
  if (kList && !kEarly && tid == 0) s_next_item = next_ticket + int(gridDim.x);
#if WY_TRACE
  tr2 = __builtin_amdgcn_s_memrealtime();
#endif
  float l = row_sum2(l_part);
  // Some score exceeded its row's first-tile maximum by a factor over 2^64
  // (or is not finite): l is then at least 2^64.
  const bool over = qrow < n && !(l < kHeadroomScale);
  // workgroup vote: one flag per wave in LDS, as inline asm (see kEarly)
  ds_write_b32_at<0>(lds_u32(reinterpret_cast<unsigned char *>(s_over)) + uint32_t(wave * 4),
                     __ballot(over) != 0 ? 1u : 0u);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  u32x4_t votes = ds_read_b128_at<0>(lds_u32(reinterpret_cast<unsigned char *>(s_over)));
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(votes)::"memory");
  if (__builtin_amdgcn_readfirstlane(votes[0] | votes[1] | votes[2] | votes[3]) != 0) {
    // Cold path: some score exceeded the first tile's max by more than
    // 2^64.  Redo the block exactly: a max pass, then accumulation.
    issue_first();
    run_pass(std::integral_constant<int, 1>{});
    __syncthreads();
    issue_first();
    zero_acc();
    run_pass(std::integral_constant<int, 2>{});
    l = row_sum2(l_part);
    if constexpr (kEarly) {
      // the passes reused the K ring and the q registers: request the next
      // block's again
      __syncthreads();
      if (npf) load_q_rows(nstart, nn, nqb * kBQ, nh);
      prefetch_k();
    }
  }

  // ---- normalise and store: lane holds row qrow, dims dt*32 + 8j + 4g + i -------
  // The block's output is 32 rows of 4 heads x 256 dims, each row one 2 KiB
  // run in memory.  The lanes' 8-byte pieces (16 bytes of each row per store
  // instruction) are staged in LDS and written back as whole rows: each store
  // instruction then covers 1 KiB of one row instead of 32 rows.
  const float inv_l = 1.0f / l;
  // every wave is past its last K/V read of the rings (LDS order only)
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#if WY_TRACE
  tre = __builtin_amdgcn_s_memrealtime();
#endif
  // Queue launch: the next block's coordinates, q rows and K tiles 0 and 1
  // are requested before the last tile's PV (kEarly) or, in the attention
  // block, after the staging reads (its gate registers are free then); its V
  // tile 0 once every wave has read the output staging out of that ring
  // slot; all before this block's output stores.  The staging's LDS accesses
  // are inline asm: the compiler cannot tell a DMA's LDS target from theirs
  // and would make them wait for it.
#if WY_TRACE
  tpf = __builtin_amdgcn_s_memrealtime();
#endif
  bf16_t *const stage = reinterpret_cast<bf16_t *>(v_ring);
  {
    const uint32_t sw = lds_u32(reinterpret_cast<unsigned char *>(stage + col * kStagePitch +
                                                                  wave * kD + 4 * g));
    static_for<0, 8>([&](auto dtc) {
      constexpr int dt = decltype(dtc)::value;
      static_for<0, 4>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const u32x2_t w = {pack_bf16x2(o[dt][4 * j] * inv_l, o[dt][4 * j + 1] * inv_l),
                           pack_bf16x2(o[dt][4 * j + 2] * inv_l, o[dt][4 * j + 3] * inv_l)};
        ds_write_b64_at<(dt * 32 + 8 * j) * 2>(sw, w);
      });
    });
  }
#if WY_TRACE
  tsw = __builtin_amdgcn_s_memrealtime();
#endif
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  {
    // 256 threads x 16 bytes = two rows per step; thread tid keeps its column
#if WY_TRACE
    trs = __builtin_amdgcn_s_memrealtime();
#endif
    const int rows = min(kBQ, n - q0);
    const uint32_t sp = lds_u32(reinterpret_cast<unsigned char *>(stage + r0 * kStagePitch + c8));
    u32x4_t wv[kBQ / 2];
    static_assert(kBQ == 32, "16 staging reads");
    static_for<0, kBQ / 2>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      wv[i] = ds_read_b128_at<i * 2 * kStagePitch * 2>(sp);
    });
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(wv[0]), "+v"(wv[1]), "+v"(wv[2]), "+v"(wv[3]), "+v"(wv[4]), "+v"(wv[5]),
                   "+v"(wv[6]), "+v"(wv[7]), "+v"(wv[8]), "+v"(wv[9]), "+v"(wv[10]), "+v"(wv[11]),
                   "+v"(wv[12]), "+v"(wv[13]), "+v"(wv[14]), "+v"(wv[15])::"memory");
#pragma unroll
    for (int i = 0; i < kBQ / 2; ++i) {
      if constexpr (kRot > 0) {
        // bf16(ctx * sigmoid(gate)), ctx the bf16 attention output, as the
        // gate pack computes it
#pragma unroll
        for (int e = 0; e < 4; ++e)
          wv[i][e] = pack_bf16x2(bf16_lo(wv[i][e]) * gate_sigmoid(bf16_lo(gate_c[i][e])),
                                 bf16_hi(wv[i][e]) * gate_sigmoid(bf16_hi(gate_c[i][e])));
      }
    }
    if constexpr (kList && kRot > 0) prefetch_q();  // the gate registers are free now
    if constexpr (kList) {
      if (!kEarly && npf) {
        const __amdgpu_buffer_rsrc_t nk = mk_rsrc(k, ks_t, ks_h, nstart, nn, nh, k_row_bytes);
        dma_k(nk, 0, 0, 0, kKPerWave);
        if (ntiles > 1) dma_k(nk, 1, 1, 0, kKPerWave);
      }
      // Buffer stores whose range ends after row `rows` - 1 (a row past it
      // lies beyond the range, the launch checks the strides), so that every
      // thread issues exactly 16 stores.
      bf16_t *const ob0 = out + (int64_t(start) + q0) * os_t + (h * kG) * os_h;
      const __amdgpu_buffer_rsrc_t o_rsrc = __builtin_amdgcn_make_buffer_rsrc(
          ob0, 0,
          int(uint32_t(rows - 1) * uint32_t(os_t) * 2u + uint32_t(kG - 1) * uint32_t(os_h) * 2u +
              kD * 2),
          0x00020000);
      const uint32_t o_voff = uint32_t(r0) * uint32_t(os_t) * 2u +
                              uint32_t(c8 / kD) * uint32_t(os_h) * 2u + uint32_t(c8 % kD) * 2u;
      // Every wave is past its last read of the output staging before the
      // next block's V(0) lands in its slot (zeroed first when that block's
      // last tile is partial: rows past the sequence must hold finite
      // values).  Only LDS order matters here: a bare barrier after the LDS
      // counter, since a __syncthreads fence would also wait for the
      // prefetched loads.  V(0) goes out before the stores, so the next
      // block's first wait leaves only the stores in flight.
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (npf) {
        if (nn < ntiles * kBN) {
          // as inline asm: the compiler would make these wait for the K DMAs
          const uint32_t zb = lds_u32(v_ring) + uint32_t(tid * 16);
          const u32x4_t z = {0u, 0u, 0u, 0u};
          static_assert(2 * kTileV % (256 * 16) == 0 && 2 * kTileV / (256 * 16) == 18,
                        "V ring zeroing");
          static_for<0, 9>([&](auto ic) {
            ds_write_b128_at<decltype(ic)::value * 4096>(zb, z);
            ds_write_b128_at<decltype(ic)::value * 4096>(zb + 9 * 4096, z);
          });
          asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
        // as inline asm: the next block's prologue reads the plan in LDS,
        // and the compiler would make those reads wait for this DMA (and, by
        // the in-order counter, for everything requested before it)
        const __amdgpu_buffer_rsrc_t nv = mk_rsrc(v, vs_t, vs_h, nstart, nn, nh, v_row_bytes);
#pragma unroll
        for (int i = 0; i < kVPerWave; ++i)
          dma16_lds_asm(nv, lds_u32(v_ring + (wave + 4 * i) * 1024), v_voff[i], 0u);
      }
#pragma unroll
      for (int i = 0; i < kBQ / 2; ++i)
        __builtin_amdgcn_raw_buffer_store_b128(wv[i], o_rsrc, o_voff,
                                               uint32_t(2 * i) * uint32_t(os_t) * 2u, 2);
    } else {
      bf16_t *ob = out + (int64_t(start) + q0 + r0) * os_t + (h * kG + c8 / kD) * os_h + c8 % kD;
#pragma unroll
      for (int i = 0; i < kBQ / 2; ++i) {
        if (r0 + 2 * i < rows) st16_nt(ob, wv[i]);
        ob += 2 * os_t;
      }
    }
  }
#if WY_TRACE
  if (tid == 0 && blockIdx.x < 256 && trace_k < 64) {
    unsigned long long *tp = g_trace + (blockIdx.x * 64 + trace_k) * 8;
    unsigned hw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    tp[0] = tr0; tp[1] = tr1; tp[2] = tr2; tp[3] = __builtin_amdgcn_s_memrealtime();
    tp[4] = (unsigned long long)(b) | ((unsigned long long)qb << 16) | ((unsigned long long)h << 32);
    tp[5] = n_tiles | ((trm - tr0) << 8) | ((trq - tr0) << 24) | ((tre - tr2) << 40);
    tp[6] = (trs - tr2) | ((tpf - tr2) << 16) | ((tsw - tr2) << 32); tp[7] = 1;
  }
  ++trace_k;
#endif
  if constexpr (!kList) return;
  item = nitem;
  b = nb;
  h = nh;
  qb = nqb;
  pf = npf;
  }
}

}  // namespace wy_prefill
