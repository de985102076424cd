// Packed varlen causal GQA prefill for short sequences (every sequence at
// most two 64-token KV tiles long) whose query blocks fit the chip in one
// round: the direct launch of 32 x 128-token prompts and the like.
//
// Such a launch is latency-bound, not MFMA- or HBM-bound: every CU holds one
// block, every block loads its q rows and K/V at once, computes, and stores,
// and the four-wave kernel runs its block's QK -> softmax -> PV chain on one
// wave per SIMD with the memory system idle meanwhile.  Here a block (the same
// sequence, KV head and 32-token query block as in prefill_kernel.h) runs on
// eight waves, a pair per query head, so each SIMD holds two waves whose
// chains interleave:
//   * S^T: score slab j holds keys 32j .. 32j+31; query block qb sees slabs
//     0 .. qb (slab qb is the diagonal one, the later ones are fully masked
//     and skipped), and wave half hf scores slabs hf and hf + 2 (K from LDS,
//     q from LDS, where the block's rows were staged by DMA);
//   * the row max is exact over the whole block (the halves swap their
//     partial maxima through LDS), so no score can outgrow the reference and
//     the four-wave kernel's exact two-pass path is not needed;
//   * the scores come out of the MFMAs unscaled (raw q rows as the B
//     operand); 1/sqrt(D) in log2 units enters the exponentials' fused
//     multiply-add, so the VALU never rescales q (a wave64 VALU instruction
//     takes four cycles: rescaling and re-rounding q cost more than the
//     block's MFMAs);
//   * P (bf16, exactly as the reference rounds it) is swapped through LDS, and
//     each half accumulates O^T for 128 of the 256 dims over every visible
//     slab;
//   * the row sum l is the halves' partial sums added in half order, so both
//     waves of a pair normalise with the same l.
// Results agree with the four-wave kernel to rounding (the same math, with
// the scale applied to the scores instead of to a bf16-rounded q, and an
// exact row max as the exponentials' reference); the launch chooses this kernel
// by the shape alone, so a given input always takes the same kernel.
//
// The LDS holds the rings of prefill_kernel.h (two K slots, two V slots; V
// rows padded for the transposing reads), with q and K rows in the paired
// layout below; tiles land by LDS DMA, and every LDS access is inline asm with
// explicit waits, so the compiler adds no wait for the DMAs before them.
#include "prefill_kernel.h"

namespace wy_prefill {

constexpr int kSWaves = 8;
constexpr int kSVPerWave = (kVDma + kSWaves - 1) / kSWaves;  // 5 (40 >= 36 blocks)
// q and K rows in LDS: groups of 32 rows; rows r and r + 16 of a group share
// one 1040-byte pair slot (r at +0, r + 16 at +512), pair slots of a group
// 1040 bytes apart.  One 1 KiB LDS DMA then fills a pair slot with lane-
// invariant offsets (lane l: row r + 16 (l / 32), chunk l % 32), and the
// operand reads of 16 consecutive rows start 65 16-byte bank groups apart
// (conflict-free).
constexpr int kPairPitch = 1040;
constexpr int kGroupBytes = 16 * kPairPitch;  // 32 rows
static_assert(2 * kGroupBytes <= kTileK, "a K tile of two row groups fits its slot");
// q staging: 4 heads x 32 rows, one group per head, in the V ring
constexpr int kQRows = kG * kBQ;
static_assert(kG * kGroupBytes <= 2 * kTileV, "q staging fits the V ring");
// LDS offset of row r of a group-layout tile
__host__ __device__ constexpr int grow_off(int r) {
  return (r >> 5) * kGroupBytes + (r & 15) * kPairPitch + ((r >> 4) & 1) * 512;
}
static_assert(64 * kSWaves * kSVPerWave <= 2560,
              "V DMA slot indices in the range where div36 is exact");
// P exchange in the K ring once every wave is past its S^T: per wave two
// units of two 1 KiB k-step blocks.
constexpr int kXchWave = 4096;

#if WY_TRACE
// per-block phase stamps (s_memrealtime at 100 MHz; s_memtime cycles), 32 slots per block
namespace {
__device__ unsigned long long g_strace[4096 * 32];
}  // namespace
#define WY_STAMP(i)                                                     \
  do {                                                                  \
    unsigned long long t_ = __builtin_amdgcn_s_memrealtime();           \
    asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(t_)::"memory");          \
    unsigned long long c_ = __builtin_amdgcn_s_memtime();               \
    asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(c_)::"memory");          \
    if (tid == 0 && blockIdx.x < 4096) {                                \
      g_strace[blockIdx.x * 32 + (i)] = t_;                             \
      if ((i) >= 2 && (i) <= 5) g_strace[blockIdx.x * 32 + 7 + (i)] = c_; \
    }                                                                   \
  } while (0)
#define WY_CSTAMP(i)                                                    \
  do {                                                                  \
    unsigned long long c_ = __builtin_amdgcn_s_memtime();               \
    asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(c_)::"memory");          \
    if (tid == 0 && blockIdx.x < 4096) g_strace[blockIdx.x * 32 + (i)] = c_; \
  } while (0)
#else
#define WY_CSTAMP(i) \
  do {               \
  } while (0)
#define WY_STAMP(i) \
  do {              \
  } while (0)
#endif

// Per-lane V DMA offsets with 24-bit multiplies (full rate; a 32-bit
// multiply takes four VALU slots): the launch checks that the V row stride
// is below 2^24 bytes.  x / 36 as a multiply-shift, exact for x < 2560.
__device__ __forceinline__ uint32_t div36(uint32_t x) { return __umul24(x, 1821u) >> 16; }

__device__ __forceinline__ uint32_t ds_read_b32_at(uint32_t addr) {
  uint32_t r;
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
static_assert(kSWaves * kXchWave <= 2 * kTileK, "P exchange fits the K ring");

template <int kRot>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void short_prefill_kernel(
    const bf16_t *__restrict__ q, int64_t qs_t, int64_t qs_h,
    const bf16_t *__restrict__ k, int64_t ks_t, int64_t ks_h,
    const bf16_t *__restrict__ v, int64_t vs_t, int64_t vs_h, bf16_t *__restrict__ out,
    int64_t os_t, int64_t os_h, const int32_t *__restrict__ cu, float qk_scale_log2, int n_seq,
    int n_kv_heads, int n_qblocks, const BlockArgs blk, int ticket_order) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ __align__(16) float s_mx[kSWaves * 64];
  __shared__ __align__(16) float s_ps[kSWaves * 64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hd = wave & 3;   // query head within the GQA group
  const int hf = wave >> 2;  // half of the pair
  const int g = lane >> 5;
  const int col = lane & 31;

  unsigned char *const k_ring = smem;
  unsigned char *const v_ring = smem + 2 * kTileK;

  // Block of this workgroup: heaviest first, as the four-wave direct launch
  // (test hook: ticket_order permutes the same blocks).
  const int bh_count = n_seq * n_kv_heads;
  int it = int(blockIdx.x);
  const int n_items = int(gridDim.x);
  if (ticket_order == 1) it = n_items - 1 - it;
  else if (ticket_order == 2) it = (it & 1) ? n_items - 1 - (it >> 1) : (it >> 1);
  const int slice = it / bh_count;
  const int bh = it - slice * bh_count;
  const int b = bh / n_kv_heads;
  const int h = bh - b * n_kv_heads;
  const int qb = n_qblocks - 1 - slice;
  const int start = cu[b];
  const int n = cu[b + 1] - start;
  const int q0 = qb * kBQ;
  if (q0 >= n) return;  // uniform over the workgroup
  WY_STAMP(0);
  const int qrow = q0 + col;
  const int kv_end = min(q0 + kBQ, n);
  const int n_tiles = (kv_end + kBN - 1) / kBN;  // 1 or 2 (the launch checks)
  const int row_lim = min(qrow, n - 1);

  // ---- requests: (RoPE table,) q rows, K tiles, V tiles -------------------
  // Issued in this order with a fixed count per wave, so that each wait
  // below counts exactly the younger requests it leaves in flight.
  // Attention block: sin / cos of the q rows' RoPE (the K/V launch's table).
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
  // q: the block's 32 rows of its 4 heads, whole rows by LDS DMA into the V
  // ring (128 rows padded like K rows: the slice reads below are then
  // conflict-free), read back as each lane's 16-byte slices; the V tiles
  // follow once every wave has read its slices.  (Loaded straight into the
  // lanes' slices, each q load instruction touched 32 rows, and the K DMAs
  // queued behind them.)  The buffer range ends after the last row's fourth
  // head: rows past the sequence read bytes of q that are never used.
  const uint32_t q_row_b = uint32_t(qs_t) * 2u, q_head_b = uint32_t(qs_h) * 2u;
  const __amdgpu_buffer_rsrc_t q_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t *>(q + (int64_t(start) + q0) * qs_t + (h * kG) * qs_h), 0,
      int(uint32_t(n - 1 - q0) * q_row_b + uint32_t(kG - 1) * q_head_b + kD * 2), 0x00020000);
  unsigned char *const dummy = smem + kRingBytes;
  // pair slot p of head group hq: rows (tokens) p and p + 16
  const uint32_t lane_chunk = uint32_t(lane & 31) * 16u;
  const uint32_t q_voff = uint32_t(lane >> 5) * 16u * q_row_b + lane_chunk;
#pragma unroll
  for (int i = 0; i < kQRows / 2 / kSWaves; ++i) {
    const int ps = wave + kSWaves * i;  // pair slot 0..63: head ps / 16, token ps % 16
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        q_rsrc, (lds_void_t *)(v_ring + (ps >> 4) * kGroupBytes + (ps & 15) * kPairPitch), 16,
        q_voff, uint32_t(ps & 15) * q_row_b + uint32_t(ps >> 4) * q_head_b, 0, 0);
  }
  const uint32_t k_row_bytes = uint32_t(ks_t) * 2u;
  const uint32_t v_row_bytes = uint32_t(vs_t) * 2u;
  const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t *>(k + int64_t(start) * ks_t + h * ks_h), 0,
      int(uint32_t(n - 1) * k_row_bytes + kD * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t *>(v + int64_t(start) * vs_t + h * vs_h), 0,
      int(uint32_t(n - 1) * v_row_bytes + kD * 2), 0x00020000);
  // Both tiles' DMAs are always issued (a fixed request count); in a
  // one-tile block the second tile's offset lies past the buffer range, so
  // nothing is fetched (and its ring slots are not read).  K row r of a tile
  // holds token k_row_token(r); rows r and r + 16 of a group hold tokens 8
  // apart.
  const uint32_t k_voff = uint32_t(lane >> 5) * 8u * k_row_bytes + lane_chunk;
  static_for<0, 2>([&](auto tc) {
    constexpr int t = decltype(tc)::value;
#pragma unroll
    for (int i = 0; i < kBN / 2 / kSWaves; ++i) {
      const int ps = wave + kSWaves * i;  // pair slot 0..31: group ps / 16, rows ps % 16 (+16)
      const int r = 32 * (ps >> 4) + (ps & 15);
      const uint32_t soff =
          t < n_tiles ? uint32_t(t * kBN + k_row_token(r)) * k_row_bytes : 0x40000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          k_rsrc, (lds_void_t *)(k_ring + t * kTileK + grow_off(r)), 16, k_voff, soff, 0, 0);
    }
  });
  // The V DMAs' per-lane offsets, computed while the q rows and K tiles are
  // in flight (the asm pins them here, off the path from the q slices to
  // the first S^T MFMA).
  uint32_t v_voff[kSVPerWave];
#pragma unroll
  for (int i = 0; i < kSVPerWave; ++i) {
    const uint32_t sl = uint32_t(64 * (wave + kSWaves * i) + lane);
    const uint32_t row = div36(sl);
    const uint32_t c = sl - row * kVSlots;
    v_voff[i] = __umul24(row < kBN ? row : kBN - 1, v_row_bytes) + (c < kD / 8 ? c : 0) * 16u;
  }
  static_assert(kSVPerWave == 5, "pinned V offsets");
  asm volatile("" : "+v"(v_voff[0]), "+v"(v_voff[1]), "+v"(v_voff[2]), "+v"(v_voff[3]),
               "+v"(v_voff[4]));
  // q rows and K tiles landed (this wave's DMAs), then every wave's
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  WY_STAMP(1);
  u32x4_t xr[16];
  {
    const uint32_t qr = lds_u32(v_ring) + uint32_t(grow_off(hd * kBQ + col) + g * 16);
    static_for<0, 16>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      xr[i] = ds_read_b128_at<i * 32>(qr);
    });
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(xr[0]), "+v"(xr[1]), "+v"(xr[2]), "+v"(xr[3]), "+v"(xr[4]), "+v"(xr[5]),
                   "+v"(xr[6]), "+v"(xr[7]), "+v"(xr[8]), "+v"(xr[9]), "+v"(xr[10]), "+v"(xr[11]),
                   "+v"(xr[12]), "+v"(xr[13]), "+v"(xr[14]), "+v"(xr[15])::"memory");
  }
  // every wave has its slices: the V tiles may land in the ring
  asm volatile("s_barrier" ::: "memory");
  // The V rows past the sequence's end are not fetched; their P is 0 but
  // their LDS rows must hold finite values: this wave zeroes the blocks it
  // is about to fill of a partial last tile (its own zero writes complete
  // before its DMA is issued).
  if (n < n_tiles * kBN) {
    const uint32_t vz = lds_u32(v_ring + (n_tiles - 1) * kTileV) + uint32_t(lane * 16);
    const u32x4_t z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < kSVPerWave; ++i)
      if (wave + kSWaves * i < kVDma)
        asm volatile("ds_write_b128 %0, %1 offset:0" ::"v"(vz + uint32_t((wave + kSWaves * i) * 1024)),
                     "v"(z)
                     : "memory");
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
  static_for<0, 2>([&](auto tc) {
    constexpr int t = decltype(tc)::value;
    const uint32_t soff = t < n_tiles ? uint32_t(t * kBN) * v_row_bytes : 0x40000000u;
#pragma unroll
    for (int i = 0; i < kSVPerWave; ++i) {
      const int blk_i = wave + kSWaves * i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          v_rsrc, (lds_void_t *)(blk_i < kVDma ? v_ring + t * kTileV + blk_i * 1024 : dummy), 16,
          v_voff[i], soff, 0, 0);
    }
  });

  WY_STAMP(2);

  if constexpr (kRot > 0) {
    // the standalone kernel's device math and bf16 rounding
    // (partial_rope.py:74-98): k-step kk < kRot/32 holds dims 16kk + 8g .. +7
    // of the first half, k-step kk + kRot/32 their partners
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
  // The q rows enter the MFMAs as they are; the scale (1/sqrt(D) in log2
  // units) is applied to the scores inside the exponentials' fused
  // multiply-add.  (Scaling and re-rounding the q slices cost ~1300 VALU
  // cycles per wave -- a wave64 VALU instruction takes 4 -- twice per head
  // here, more than the block's MFMAs.)  Rows past the sequence hold finite
  // q bytes (or zeros) and only reach their own, unstored, output rows.
  bf16x8_t qop[16];
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) qop[kk] = __builtin_bit_cast(bf16x8_t, xr[kk]);

  WY_CSTAMP(16);
  // ---- S^T of this wave's slabs ----------------------------------------------
  // Score slabs: slab j holds keys 32j .. 32j + 31 (tile j / 2, rows 32 (j % 2)
  // .. of its K slot).  The block's rows see slabs 0 .. qb; slab qb holds the
  // diagonal (and the sequence end), the earlier ones are fully visible, the
  // later ones fully masked and skipped (their P is exactly 0, so skipping
  // their MFMAs changes no bit).  Wave half hf takes slabs hf and hf + 2:
  // unit u = slab hf + 2u = (tile u, K rows 32 hf ..).
  const int n_own = hf <= qb ? (qb - hf) / 2 + 1 : 0;  // 0, 1 or 2 (uniform)
  const int n_oth = (1 - hf) <= qb ? (qb - 1 + hf) / 2 + 1 : 0;
  // (accumulators are not zeroed: each chain's first MFMA takes a zero C
  // operand -- a wave64 VALU instruction costs four cycles, and zeroing the
  // S and O accumulators took about 100 of them)
  f32x16_t s[2];
  const f32x16_t zacc = {};
  {
    const uint32_t kr = lds_u32(k_ring) + uint32_t(grow_off(32 * hf + col) + g * 16);
    if (n_own == 2) {
      // the two units alternate (independent accumulators)
      constexpr int kKW = 8;  // K operands in flight (12 and 15 measured no faster)
      u32x4_t ka[kKW];
      auto rd = [&](auto ic) {
        constexpr int i = decltype(ic)::value;  // MFMA i: unit i & 1, k-step i >> 1
        constexpr int off = (i & 1) * kTileK + (i >> 1) * 32;
        return ds_read_b128_at<off>(kr);
      };
      static_for<0, kKW>([&](auto ic) { ka[ic] = rd(ic); });
      static_for<0, 32>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        lgkm_wait1<(i + kKW <= 32 ? kKW - 1 : 31 - i)>(ka[i % kKW]);
        s[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, ka[i % kKW]),
                                                           qop[i >> 1], i < 2 ? zacc : s[i & 1],
                                                           0, 0, 0);
        if constexpr (i + kKW < 32) ka[i % kKW] = rd(std::integral_constant<int, i + kKW>{});
      });
    } else if (n_own == 1) {
      u32x4_t ka[16];
      static_for<0, 16>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        ka[i] = ds_read_b128_at<i * 32>(kr);
      });
      static_for<0, 16>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        lgkm_wait1<15 - i>(ka[i]);
        s[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, ka[i]),
                                                       qop[i], i == 0 ? zacc : s[0], 0, 0, 0);
      });
    }
  }
  WY_CSTAMP(17);
  // mask the diagonal slab (keys past the row's causal limit or the sequence
  // end); row max over this wave's slabs
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    if (u < n_own) {
      if (hf + 2 * u == qb) {
        const int thr = row_lim - (32 * qb + 16 * g);  // keep registers e <= thr
#pragma unroll
        for (int e = 0; e < 16; ++e) s[u][e] = e > thr ? -INFINITY : s[u][e];
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[u][e]);
    }
  }
  {
    float lo, hi;
    row_halves(mx, lo, hi);
    mx = fmaxf(lo, hi);
  }
  WY_CSTAMP(18);
  // (LDS accesses as inline asm here and below: the compiler would make a
  // visible one wait for every DMA it knows of, the V tiles included)
  const uint32_t mx_a = lds_u32(reinterpret_cast<unsigned char *>(s_mx));
  ds_write_b32_at<0>(mx_a + uint32_t((wave * 64 + lane) * 4), __float_as_uint(mx));
  // every wave's partial max written, and every wave past its last K read
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  WY_CSTAMP(19);
  uint32_t mx_o = ds_read_b32_at(mx_a + uint32_t(((wave ^ 4) * 64 + lane) * 4));
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(mx_o)::"memory");
  const float m = fmaxf(mx, __uint_as_float(mx_o));  // raw score units
  const float neg_ms = -(m * qk_scale_log2);
  WY_STAMP(3);

  // ---- P (bf16) of this wave's units, its row sum; swap P with the pair -----
  // Unit u's P^T B operands: k-steps kk = 0, 1 = keys 32 j + 16 g + 8 kk .. +7
  // of its slab j.
  u32x4_t pown[2][2];
  float psum = 0.f;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    if (u < n_own) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float a = __builtin_amdgcn_exp2f(__fmaf_rn(s[u][8 * kk + 2 * w], qk_scale_log2, neg_ms));
          const float c =
              __builtin_amdgcn_exp2f(__fmaf_rn(s[u][8 * kk + 2 * w + 1], qk_scale_log2, neg_ms));
          psum += a + c;
          pown[u][kk][w] = pack_bf16x2(a, c);
        }
    }
  }
  const uint32_t ps_a = lds_u32(reinterpret_cast<unsigned char *>(s_ps));
  ds_write_b32_at<0>(ps_a + uint32_t((wave * 64 + lane) * 4), __float_as_uint(psum));
  const uint32_t xw = lds_u32(k_ring) + uint32_t(wave * kXchWave + lane * 16);
  if (n_own >= 1) {
    ds_write_b128_at<0>(xw, pown[0][0]);
    ds_write_b128_at<1024>(xw, pown[0][1]);
  }
  if (n_own == 2) {
    ds_write_b128_at<2048>(xw, pown[1][0]);
    ds_write_b128_at<3072>(xw, pown[1][1]);
  }
  // V tiles landed (this wave's DMAs), the P and psum writes done; then every
  // wave's
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  const uint32_t xp = lds_u32(k_ring) + uint32_t((wave ^ 4) * kXchWave + lane * 16);
  u32x4_t poth[2][2];
  if (n_oth >= 1) {
    poth[0][0] = ds_read_b128_at<0>(xp);
    poth[0][1] = ds_read_b128_at<1024>(xp);
  }
  if (n_oth == 2) {
    poth[1][0] = ds_read_b128_at<2048>(xp);
    poth[1][1] = ds_read_b128_at<3072>(xp);
  }
  uint32_t ps_ob = ds_read_b32_at(ps_a + uint32_t(((wave ^ 4) * 64 + lane) * 4));
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(poth[0][0]), "+v"(poth[0][1]), "+v"(poth[1][0]), "+v"(poth[1][1]),
                 "+v"(ps_ob)::"memory");
  const float ps_o = __uint_as_float(ps_ob);
  WY_STAMP(4);
  // l: the halves' partial sums in half order (the same bits in both waves)
  float l = hf == 0 ? psum + ps_o : ps_o + psum;
  {
    float lo, hi;
    row_halves(l, lo, hi);
    l = lo + hi;
  }

  // ---- O^T += V^T P^T over the visible slabs, dims 128 hf .. +127 ----------
  // A operand of slab j, k-step kk, dim block dt: lane (m = lane % 32, g)
  // needs V[32 j + 16 g + 8 kk + 0..7][32 dt + m] of tile j / 2 (transposing
  // reads, as in prefill_kernel.h).
  const int l16 = lane & 15;
  const uint32_t v_lane_off =
      uint32_t((16 * g + (l16 >> 2)) * kVPitch + (16 * ((lane >> 4) & 1) + 4 * (l16 & 3)) * 2) +
      uint32_t(hf * 4 * 64);
  f32x16_t o[4];  // first written by slab 0 (always visible) from a zero C
  const uint32_t vr = lds_u32(v_ring) + v_lane_off;
  auto pv_slab = [&](auto jc, const u32x4_t(&pj)[2]) {
    constexpr int j = decltype(jc)::value;
    // 8 MFMAs (kk, dt), 6 operands in flight (12 reads: lgkmcnt counts to 15)
    constexpr int kW = 6;  // (4 and 7 measured no faster)
    u32x2_t va[8][2];
    auto rd = [&](auto xc) {
      constexpr int x = decltype(xc)::value;
      constexpr int kk = x >> 2, dt = x & 3;
      constexpr int off = (j >> 1) * kTileV + (32 * (j & 1) + 8 * kk) * kVPitch + dt * 64;
      va[x][0] = ds_read_tr16<off>(vr);
      va[x][1] = ds_read_tr16<off + 4 * kVPitch>(vr);
    };
    static_for<0, kW>([&](auto xc) { rd(xc); });
    static_for<0, 8>([&](auto xc) {
      constexpr int x = decltype(xc)::value;
      constexpr int kk = x >> 2, dt = x & 3;
      constexpr int issued = x + kW < 8 ? x + kW : 8;
      lgkm_wait2<2 * (issued - x - 1)>(va[x][0], va[x][1]);
      const u32x4_t a = {va[x][0][0], va[x][0][1], va[x][1][0], va[x][1][1]};
      o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, pj[kk]),
          j == 0 && kk == 0 ? zacc : o[dt], 0, 0, 0);
      if constexpr (x + kW < 8) rd(std::integral_constant<int, x + kW>{});
    });
  };
  // slab j's P: this wave's unit j / 2 when j % 2 == hf, else the pair's
  // (a branch on the wave-uniform half, not a per-register select)
  auto pv_all = [&](auto hc) {
    constexpr int H = decltype(hc)::value;
    static_for<0, 4>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if (j <= qb) pv_slab(jc, (j & 1) == H ? pown[j >> 1] : poth[j >> 1]);
    });
  };
  if (hf == 0) pv_all(std::integral_constant<int, 0>{});
  else pv_all(std::integral_constant<int, 1>{});

  // ---- normalise, stage, store ----------------------------------------------
  // Each wave stages its own 32 rows x 128 dims (256-byte row pieces, padded
  // by 16 bytes against bank conflicts) in its own part of the V ring and
  // stores them back as whole pieces: 4 pieces per store instruction, so no
  // second barrier (a wave reads only what it wrote; LDS accesses of one
  // wave complete in order).
  constexpr int kSPitch = 128 * 2 + 16;  // bytes per staged row piece
  static_assert(kSWaves * kBQ * kSPitch <= 2 * kTileV, "per-wave staging fits the V ring");
  const int pr = lane >> 4, pc = (lane & 15) * 8;  // piece row (+ 4 i), column (bf16)
  u32x4_t gate_c[kRot > 0 ? kBQ / 4 : 1];
  if constexpr (kRot > 0) {
    // (the range ends after the last row's piece: every byte in it lies
    // inside the gate tensor; rows past the sequence are not stored)
    const uint32_t row_b = uint32_t(blk.gs_t) * 2u;
    const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16_t *>(blk.gate + (int64_t(start) + q0) * blk.gs_t + (h * kG + hd) * blk.gs_h +
                             hf * 128),
        0, int(uint32_t(n - 1 - q0) * row_b + 128 * 2), 0x00020000);
    const uint32_t vo = uint32_t(pr) * row_b + uint32_t(pc) * 2u;
#pragma unroll
    for (int i = 0; i < kBQ / 4; ++i)
      gate_c[i] = __builtin_amdgcn_raw_buffer_load_b128(gr, vo, uint32_t(4 * i) * row_b, 0);
  }
  const float inv_l = 1.0f / l;
  // every wave is past its last V read
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  WY_STAMP(5);
  unsigned char *const stage = v_ring + wave * (kBQ * kSPitch);
  {
    const uint32_t sw = lds_u32(stage + col * kSPitch + 4 * g * 2);
    static_for<0, 4>([&](auto dtc) {
      constexpr int dt = decltype(dtc)::value;
      static_for<0, 4>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const u32x2_t w = {pack_bf16x2(o[dt][4 * j] * inv_l, o[dt][4 * j + 1] * inv_l),
                           pack_bf16x2(o[dt][4 * j + 2] * inv_l, o[dt][4 * j + 3] * inv_l)};
        ds_write_b64_at<(dt * 32 + 8 * j) * 2>(sw, w);
      });
    });
  }
  {
    WY_STAMP(6);
    const int rows = min(kBQ, n - q0);
    const uint32_t sp = lds_u32(stage + pr * kSPitch + pc * 2);
    u32x4_t wv[kBQ / 4];
    static_for<0, kBQ / 4>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      wv[i] = ds_read_b128_at<i * 4 * kSPitch>(sp);
    });
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(wv[0]), "+v"(wv[1]), "+v"(wv[2]), "+v"(wv[3]), "+v"(wv[4]), "+v"(wv[5]),
                   "+v"(wv[6]), "+v"(wv[7])::"memory");
    if constexpr (kRot > 0) {
#pragma unroll
      for (int i = 0; i < kBQ / 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          // bf16(ctx * sigmoid(gate)), ctx the bf16 attention output, as the
          // gate pack computes it
          wv[i][e] = pack_bf16x2(bf16_lo(wv[i][e]) * gate_sigmoid(bf16_lo(gate_c[i][e])),
                                 bf16_hi(wv[i][e]) * gate_sigmoid(bf16_hi(gate_c[i][e])));
    }
    bf16_t *ob = out + (int64_t(start) + q0 + pr) * os_t + (h * kG + hd) * os_h + hf * 128 + pc;
#pragma unroll
    for (int i = 0; i < kBQ / 4; ++i) {
      if (pr + 4 * i < rows) st16_nt(ob, wv[i]);
      ob += 4 * os_t;
    }
#if WY_TRACE
    WY_STAMP(7);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    WY_STAMP(8);
    if (tid == 0) {
      unsigned hw, xcc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
      g_strace[blockIdx.x * 32 + 14] = (unsigned long long)n_tiles | ((unsigned long long)qb << 8) |
                                       ((unsigned long long)b << 16);
      g_strace[blockIdx.x * 32 + 15] = (unsigned long long)hw | ((unsigned long long)xcc << 32);
    }
#endif
  }
}

template __global__ void short_prefill_kernel<0>(
    const bf16_t *__restrict__, int64_t, int64_t, const bf16_t *__restrict__, int64_t, int64_t,
    const bf16_t *__restrict__, int64_t, int64_t, bf16_t *__restrict__, int64_t, int64_t,
    const int32_t *__restrict__, float, int, int, int, const BlockArgs, int);
template __global__ void short_prefill_kernel<64>(
    const bf16_t *__restrict__, int64_t, int64_t, const bf16_t *__restrict__, int64_t, int64_t,
    const bf16_t *__restrict__, int64_t, int64_t, bf16_t *__restrict__, int64_t, int64_t,
    const int32_t *__restrict__, float, int, int, int, const BlockArgs, int);

}  // namespace wy_prefill

#if WY_TRACE
extern "C" int wy_prefill_short_trace_read(void *host, size_t bytes, int clear) {
  if (clear) {
    static unsigned long long zeros[4096 * 32];
    return int(hipMemcpyToSymbol(HIP_SYMBOL(wy_prefill::g_strace), zeros, sizeof(zeros)));
  }
  return int(hipMemcpyFromSymbol(host, HIP_SYMBOL(wy_prefill::g_strace),
                                 bytes < sizeof(wy_prefill::g_strace) ? bytes : sizeof(wy_prefill::g_strace)));
}
#endif
