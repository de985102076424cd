// Paged GQA decode attention, split-K over 16-token pages (gfx950).
//
// Partial pass: one 4-wavefront workgroup per (sequence b, KV head h, split
// s).  The split's pages are dealt round-robin to the wavefronts; each wave
// keeps its own online-softmax state for the 4 query heads of the KV group, so
// one read of a K/V page serves all 4 heads.  Per page and wave:
//   * K (16 tokens x 256 dims) is loaded straight into the B operand of
//     v_mfma_f32_16x16x32_bf16 -- lane (token n = l%16, dim group g = l/16)
//     reads 16 bytes at dims 32i + 8g; q (4 heads, rows 4..15 zero, re-read
//     from LDS) is the A operand and 8 MFMAs give the 4 x 16 score tile in
//     lanes 0..15.
//   * V is read one 512-byte row per instruction (lane l: dims 4l..4l+3) and
//     P.V runs on the VALU as v_dot2_f32_bf16 over token pairs, with P rounded
//     to bf16 (the rounding the reference applies before its PV dot).
//   * The softmax max/sum reduce across the 16 token lanes with DPP row
//     rotations.
//   * Loads are software-pipelined in registers: K of the next page is
//     requested once the score MFMAs have consumed this page's K, V of the
//     next page once P.V has consumed this page's V.  Page loads are buffer
//     loads from a per-page resource, block-table entries scalar loads issued
//     one page ahead.
// After the page loop the wave states merge through LDS and one fp32
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
// The one-launch step in the balanced order raises min_pps further to
// ceil(H_kv * sum(npg) / kWorkItems), computed by every workgroup from the
// same pos, so long batches get long splits and a lone long sequence among
// short ones still gets many.
//
// Workgroup order.  The direct order gives workgroup id b + B*(h + H*s).  The
// balanced order (batches of 16..256 sequences) lists the active splits only,
// full-size splits first and the shorter last splits after them, and hands
// item k to workgroup k: the launch then runs one round of equal-sized work
// items instead of leaving holes for inactive splits, and consecutive ids --
// which the dispatcher deals round-robin over the XCDs -- carry equal page
// counts.  The order only decides where a split runs, never its pages or its
// arithmetic, so results are identical under both orders.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "wy_common.h"

using namespace wy;

namespace {

#if WY_TRACE
// per-workgroup phase stamps of the split kernel (s_memrealtime, 100 MHz)
__device__ unsigned long long g_dtrace[1024 * 16];
#define WY_DSTAMP(i)                                                        \
  do {                                                                      \
    unsigned long long t_ = __builtin_amdgcn_s_memrealtime();               \
    asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(t_)::"memory");              \
    if (threadIdx.x == 0 && blockIdx.x < 1024) g_dtrace[blockIdx.x * 16 + (i)] = t_; \
  } while (0)
#else
#define WY_DSTAMP(i) \
  do {               \
  } while (0)
#endif
constexpr int kD = 256;   // head_dim
constexpr int kG = 4;     // query heads per KV head
constexpr int kWaves = 4; // wavefronts per split workgroup

struct DecodeArgs {
  const bf16_t *q;
  int64_t qs_b, qs_h, qs_d;
  bf16_t *kc, *vc;  // written only by the fused kernel (new token's row)
  int64_t kc_p, kc_h, kc_s, vc_p, vc_h, vc_s;
  const int32_t *bt;
  int64_t bt_b;
  const int64_t *pos;
  float *mp, *lp, *ap;
  int64_t ml_b, ml_h, ml_s, a_b, a_h, a_s;
  float scale;
  int min_pps;
  int hkv;
  int batch;
  int bt_cols;  // entries per block-table row (max_pages)
  // fused step only
  const bf16_t *kn, *vn;
  int64_t kn_b, kn_h, vn_b, vn_h;
  int32_t *counters;  // [B * H_kv], zero between launches (self-resetting)
  const bf16_t *gate; // optional sigmoid gate [B, H_q, D]
  int64_t g_b, g_h, g_d;
  bf16_t *out;        // [B, H_q, D]
  int64_t o_b, o_h, o_d;
  // fused attention block only: q/k RMSNorm weights and the partial RoPE
  const bf16_t *qw, *kw;
  const float *inv_freq;
  float eps;
  int rope_dim;
  int balanced;    // workgroup order: 0 direct, 1 balanced (see the file comment)
  int two_level;   // merge more than kMergeGroup splits through groups
  int work_items;  // balanced fused order: raise the split floor to keep the
                   // active (split, KV head) items within this many (0: off)
};

__device__ __forceinline__ int split_pps(int npg, int min_pps) {
  const int p = (npg + kMaxSplits - 1) / kMaxSplits;
  return p > min_pps ? p : min_pps;
}

__device__ __forceinline__ float readlane0(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// Max / sum over each row of 16 lanes (lanes 0..15 hold the scores): DPP
// row rotations by 8, 4, 2, 1 leave the row result in every lane of the row.
template <int kRor>
__device__ __forceinline__ float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + kRor, 0xf, 0xf,
                                                    false));
}
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, row_ror<8>(v));
  v = fmaxf(v, row_ror<4>(v));
  v = fmaxf(v, row_ror<2>(v));
  v = fmaxf(v, row_ror<1>(v));
  return v;
}
__device__ __forceinline__ float sum16(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  return v;
}

// Raw buffer resource over one cache page (bounds check off: the launcher has
// validated the strides, and every offset stays inside the page).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const bf16_t *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t *>(base), 0, -1, 0x00020000);
}



// ctx = bf16(A / L), then optionally bf16(ctx * sigmoid(gate)): the same two
// roundings as the reference's combine kernel followed by its gate pack.
// The gate's bf16 values at dims d..d+3 of query head hq, as two packed pairs.
__device__ __forceinline__ u32x2_t load_gate4(const DecodeArgs &a, int b, int hq, int d) {
  const bf16_t *g = a.gate + b * a.g_b + hq * a.g_h;
  if (a.g_d == 1 && ((a.g_b | a.g_h) & 3) == 0 && (reinterpret_cast<uintptr_t>(a.gate) & 7) == 0)
    return *reinterpret_cast<const u32x2_t *>(g + d);
  return u32x2_t{uint32_t(g[d * a.g_d]) | (uint32_t(g[(d + 1) * a.g_d]) << 16),
                 uint32_t(g[(d + 2) * a.g_d]) | (uint32_t(g[(d + 3) * a.g_d]) << 16)};
}

// gpre: the gate values, already loaded (else they are loaded here).
__device__ __forceinline__ void store_out4(const DecodeArgs &a, int b, int hq, int d,
                                           float4 A, float L, const u32x2_t *gpre = nullptr) {
  float o[4] = {round_bf16(A.x / L), round_bf16(A.y / L), round_bf16(A.z / L),
                round_bf16(A.w / L)};
  if (a.gate) {
    const u32x2_t gw = gpre ? *gpre : load_gate4(a, b, hq, d);
    o[0] *= gate_sigmoid(bf16_lo(gw[0]));
    o[1] *= gate_sigmoid(bf16_hi(gw[0]));
    o[2] *= gate_sigmoid(bf16_lo(gw[1]));
    o[3] *= gate_sigmoid(bf16_hi(gw[1]));
  }
  bf16_t *orow = a.out + b * a.o_b + hq * a.o_h;
  if (a.o_d == 1) {
    const u32x2_t w = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    *reinterpret_cast<u32x2_t *>(orow + d) = w;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) orow[(d + e) * a.o_d] = bf16_t(f32_to_bf16_bits(o[e]));
  }
}

// Device-coherent (agent-scope) scalar / 8-byte accesses.  On gfx950 each
// XCD has its own L2, so split partials handed from one workgroup to another
// inside a launch go through these instead of plain cached accesses; no
// cache-wide writeback or invalidate is then needed.
__device__ __forceinline__ void st_coherent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent4(float *p, float4 v) {
  uint64_t *q = reinterpret_cast<uint64_t *>(p);
  __hip_atomic_store(q, (uint64_t(__float_as_uint(v.y)) << 32) | __float_as_uint(v.x),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(q + 1, (uint64_t(__float_as_uint(v.w)) << 32) | __float_as_uint(v.z),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <bool kCoherent>
__device__ __forceinline__ float ld_f(const float *p) {
  if constexpr (kCoherent)
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    return *p;
}
template <bool kCoherent>
__device__ __forceinline__ float4 ld_f4(const float *p) {
  if constexpr (kCoherent) {
    uint64_t *q = reinterpret_cast<uint64_t *>(const_cast<float *>(p));
    const uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(__uint_as_float(uint32_t(lo)), __uint_as_float(uint32_t(lo >> 32)),
                       __uint_as_float(uint32_t(hi)), __uint_as_float(uint32_t(hi >> 32)));
  } else {
    return *reinterpret_cast<const float4 *>(p);
  }
}

// Merging split states.  A state is (m, l, acc): the running max, the sum of
// exp(score - m) and the unnormalised accumulator.  One wavefront merges n
// states of one query head; lane owns dims 4*lane..4*lane+3.  The caller
// hands over lane-parallel m/l (lane i: state i, lane i+64: state i+64) and
// a function returning state i's accumulator row.  The weights are formed
// lane-parallel and the accumulator rows fetched 8 at a time, so a merge
// costs a few memory round trips rather than one per state.  The same code
// runs in the combine kernel and in the one-launch step, so both produce the
// same bits.
struct Merged {
  float M, L;
  float4 A;
};

template <class AccFn>
__device__ __forceinline__ Merged merge_core(int n, float m0, float m1, float l0, float l1,
                                             AccFn acc_row) {
  float4 x[8];
#pragma unroll
  for (int u = 0; u < 8; ++u)
    if (u < n) x[u] = acc_row(u);
  const float mx = wave_max(fmaxf(m0, m1));
  const float w0 = m0 == -INFINITY ? 0.f : __expf(m0 - mx);
  const float w1 = m1 == -INFINITY ? 0.f : __expf(m1 - mx);
  const float L = wave_sum(w0 * l0 + w1 * l1);
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < n; s0 += 8) {
    if (s0 > 0) {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < n) x[u] = acc_row(s0 + u);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int sp = s0 + u;
      if (sp < n) {
        const float w = __shfl(sp < 64 ? w0 : w1, sp & 63);
        A.x += w * x[u].x;
        A.y += w * x[u].y;
        A.z += w * x[u].z;
        A.w += w * x[u].w;
      }
    }
  }
  return Merged{mx, L, A};
}

// Merge n states of (b, hq) stored in the scratch at slots first + i*stride.
// kCoherent: they were published by other workgroups of this launch.
template <bool kCoherent>
__device__ Merged merge_slots(const DecodeArgs &a, int b, int hq, int first, int stride, int n,
                              int lane) {
  const float *mrow = a.mp + b * a.ml_b + hq * a.ml_h;
  const float *lrow = a.lp + b * a.ml_b + hq * a.ml_h;
  const float *arow = a.ap + b * a.a_b + hq * a.a_h + lane * 4;
  const bool has0 = lane < n, has1 = lane + 64 < n;
  const int s0 = first + lane * stride, s1 = first + (lane + 64) * stride;
  const float m0 = has0 ? ld_f<kCoherent>(mrow + s0 * a.ml_s) : -INFINITY;
  const float m1 = has1 ? ld_f<kCoherent>(mrow + s1 * a.ml_s) : -INFINITY;
  const float l0 = has0 ? ld_f<kCoherent>(lrow + s0 * a.ml_s) : 0.f;
  const float l1 = has1 ? ld_f<kCoherent>(lrow + s1 * a.ml_s) : 0.f;
  return merge_core(n, m0, m1, l0, l1, [&](int i) {
    return ld_f4<kCoherent>(arow + (first + i * stride) * a.a_s);
  });
}

// Splits per merge group.  Up to kMergeGroup splits merge in one level (the
// last split of the sequence and KV head to finish merges them all); with
// two_level set (a long sequence cut into up to 128 splits) more merge in
// two: the last split of each group of
// kMergeGroup merges its group into the group's first slot, and the last
// group to finish merges the group states.  One merging wavefront then reads
// at most 16 accumulator rows (16 KiB) instead of up to 128.
constexpr int kMergeGroup = 16;

// Merge all nact split states of (b, hq) as the one-launch step does.
template <bool kCoherent>
__device__ Merged merge_all(const DecodeArgs &a, int b, int hq, int nact, int lane) {
  if (!a.two_level || nact <= kMergeGroup)
    return merge_slots<kCoherent>(a, b, hq, 0, 1, nact, lane);
  const int ng = (nact + kMergeGroup - 1) / kMergeGroup;  // <= 8
  float mg = -INFINITY, lg = 0.f;
  float4 ag[kMaxSplits / kMergeGroup];
#pragma unroll
  for (int g = 0; g < kMaxSplits / kMergeGroup; ++g) {
    ag[g] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (g < ng) {
      const Merged r = merge_slots<kCoherent>(a, b, hq, g * kMergeGroup, 1,
                                              min(kMergeGroup, nact - g * kMergeGroup), lane);
      if (lane == g) {
        mg = r.M;
        lg = r.L;
      }
      ag[g] = r.A;
    }
  }
  return merge_core(ng, mg, -INFINITY, lg, 0.f, [&](int i) {
    float4 v = ag[0];
#pragma unroll
    for (int g = 1; g < kMaxSplits / kMergeGroup; ++g)
      if (i == g) v = ag[g];
    return v;
  });
}

// Balanced workgroup order: work item k (k = blockIdx.x) of the launch.  The
// full-size splits of every (sequence, KV head) come first, sequence-major
// with the KV head and then the split index fastest, then the partial last
// splits in sequence order.  pos is read once per 64 sequences into
// registers.  Returns false for ids past the last item.
constexpr int kBalancedMinBatch = 16;
constexpr int kBalancedChunks = 4;  // batch <= 256
__device__ bool balanced_item(const DecodeArgs &a, int k, int lane, int &b, int &h, int &s,
                              int &seq_len, int &min_pps) {
  const int H = a.hkv;
  const int nch = (a.batch + 63) >> 6;
  int plo[kBalancedChunks], npg[kBalancedChunks], pps[kBalancedChunks];
#pragma unroll
  for (int c = 0; c < kBalancedChunks; ++c) {
    const int bb = c * 64 + lane;
    plo[c] = c < nch && bb < a.batch ? int(a.pos[bb]) : -1;
  }
#pragma unroll
  for (int c = 0; c < kBalancedChunks; ++c) npg[c] = (plo[c] + kPage) / kPage;
  min_pps = a.min_pps;
  if (a.work_items > 0) {
    // Split floor from the batch's total pages: ceil(H * total / work_items),
    // so the launch holds at most work_items + B*H items whatever the
    // lengths (every workgroup computes the same value from the same pos).
    int tot = 0;
#pragma unroll
    for (int c = 0; c < kBalancedChunks; ++c) tot += npg[c];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) tot += __shfl_xor(tot, o);
    const int need = int((int64_t(tot) * H + a.work_items - 1) / a.work_items);
    min_pps = __builtin_amdgcn_readfirstlane(need > min_pps ? need : min_pps);
  }
#pragma unroll
  for (int c = 0; c < kBalancedChunks; ++c) pps[c] = split_pps(npg[c], min_pps);
  int carry = 0;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int c = 0; c < kBalancedChunks; ++c) {
      if (c >= nch) break;
      const int full = npg[c] / pps[c];
      const int x = (pass == 0 ? full : int(full * pps[c] < npg[c])) * H;
      int incl = x;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
      }
      incl += carry;
      const uint64_t m = __ballot(k < incl);
      if (m) {
        const int L = __builtin_ctzll(m);
        const int r = k - __shfl(incl - x, L);
        b = __builtin_amdgcn_readfirstlane(c * 64 + L);
        h = __builtin_amdgcn_readfirstlane(r % H);
        s = __builtin_amdgcn_readfirstlane(pass == 0 ? r / H : __shfl(full, L));
        seq_len = __builtin_amdgcn_readfirstlane(__shfl(plo[c], L) + 1);
        return true;
      }
      carry = __shfl(incl, 63);
    }
  }
  return false;
}

// Split partial pass.  kFused additionally (i) takes the new token's K/V
// from k_new/v_new and writes them into their page (the append), and (ii)
// lets the last workgroup of each (b, h) to finish merge all splits and write
// the (optionally gated) output, so one launch is a whole decode step.
template <int kW>
struct SplitLds {
  u32x4_t p[kW][kPage / 2];      // bf16 P, token pairs: p[wave][j][r] = (P[r][2j], P[r][2j+1])
  float ml[kW][2][kG];           // per-wave m, l
  float4 acc[kW][kG][kD / 4];    // per-wave unnormalised acc
  bf16_t q[kG][kD + 8];          // the group's query rows
  bf16_t kn[kD];                 // fused: the new token's key (normalised, rotated in the block)
  bf16_t vn[kD];                 // fused: the new token's value
  int last;
};

// kProlog (with kFused): the decode attention block.  q and the new key
// arrive raw from the fused projection; the kernel applies the per-head
// RMSNorm (weight 1 + w) and the partial RoPE at position pos itself, with the
// same device code and roundings as the standalone qwen_rmsnorm and
// partial_rope kernels, so the block equals the op-by-op sequence bit for bit.
template <bool kFused, int kW, bool kProlog>
__global__ __launch_bounds__(64 * kW) __attribute__((amdgpu_waves_per_eu(4)))
void paged_decode_split_kernel(const DecodeArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  SplitLds<kW> &sm = *reinterpret_cast<SplitLds<kW> *>(lds_raw);
  auto &sm_p = sm.p;
  auto &sm_ml = sm.ml;
  auto &sm_acc = sm.acc;
  auto &sm_q = sm.q;

  // 1-D grid of batch * H_kv * max_splits workgroups (see the file comment
  // for the two orders).  Splits past a sequence's end exit at once.
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  typedef const __attribute__((address_space(4))) int32_t *bt_const_t;
  int b, h, s, seq_len = 0, min_pps = a.min_pps;
  if (a.balanced) {
    if (!balanced_item(a, blockIdx.x, lane, b, h, s, seq_len, min_pps)) return;
  } else {
    b = blockIdx.x % a.batch;
    h = (blockIdx.x / a.batch) % a.hkv;
    s = blockIdx.x / (a.batch * a.hkv);
  }
  const int32_t *btrow = a.bt + b * a.bt_b;
  const bt_const_t bt_s = (bt_const_t)btrow;
  const int r_q = threadIdx.x >> 5, c_q = (threadIdx.x & 31) * 8;
  const bf16_t *q_src = a.q + b * a.qs_b + (h * kG + r_q) * a.qs_h + c_q;
  const bool q_fast = threadIdx.x < kG * kD / 8 && (kProlog || a.qs_d == 1);
  u32x4_t q_pre = {0u, 0u, 0u, 0u};
  if (q_fast) q_pre = ld16(q_src);
  // The block-table entry of this wave's first page is requested together
  // with the q rows (and, in the direct order, with pos: for the usual
  // partition, pps == min_pps, its index is known before pos), so the first
  // page's address costs one memory round trip.  (pos < 2^31: its low word.)
  int32_t bt_guess;
  if (a.balanced) {
    const int npg_b = (seq_len + kPage - 1) / kPage;
    const int first = s * split_pps(npg_b, min_pps) + wave;
    bt_guess = bt_s[first < npg_b ? first : npg_b - 1];
  } else {
    const int first_guess = s * a.min_pps + wave;
    const int32_t *bt_first = btrow + (first_guess < a.bt_cols ? first_guess : a.bt_cols - 1);
    int32_t pos_lo;
    // Both outputs are early-clobber: the first load's destination must not
    // share registers with the second load's address, which is read when the
    // second load issues -- possibly after the first has returned.
    asm volatile(
        "s_load_dword %0, %2, 0x0\n\t"
        "s_load_dword %1, %3, 0x0\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(pos_lo), "=&s"(bt_guess)
        : "s"(a.pos + b), "s"(bt_first)
        : "memory");
    seq_len = pos_lo + 1;
  }
  WY_DSTAMP(1);
  const int npg = (seq_len + kPage - 1) / kPage;
  const int pps = split_pps(npg, min_pps);
  const int nact = (npg + pps - 1) / pps;
  if (s * pps >= npg) return;  // inactive split: uniform over the workgroup
  const int p0 = s * pps;
  const int p1 = min(p0 + pps, npg);

  const int n16 = lane & 15, g4 = lane >> 4;
  // The step's gate values for this wave's query head are requested up
  // front: the output epilogue then does not wait a memory round trip for them.
  u32x2_t gate_pre = {0u, 0u};
  if (kFused && a.gate && wave < kG) gate_pre = load_gate4(a, b, h * kG + wave, lane * 4);

  float m_run[kG], l_run[kG], acc[kG][4];
#pragma unroll
  for (int r = 0; r < kG; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[r][e] = 0.f;
  }

  const bf16_t *kh = a.kc + h * a.kc_h;
  const bf16_t *vh = a.vc + h * a.vc_h;
  const int last_page = (seq_len - 1) / kPage;
  const int last_slot = (seq_len - 1) % kPage;
  const bf16_t *knrow = nullptr, *vnrow = nullptr;
  if constexpr (kFused) {
    knrow = a.kn + b * a.kn_b + h * a.kn_h;
    vnrow = a.vn + b * a.vn_b + h * a.vn_h;
  }

  // This wave's pages are p0 + wave + i*kW, i < npw.  Their block-table
  // entries are read with scalar loads (the table is constant during the
  // launch), one page ahead, so a page's address never waits on the vector
  // memory counter that its K/V loads share.
  const int npw = p0 + wave < p1 ? (p1 - p0 - wave + kW - 1) / kW : 0;
  int32_t bt_ahead = npw > 0 ? (a.balanced || pps == min_pps ? bt_guess : bt_s[p0 + wave]) : 0;
  // Register pipeline, no extra registers: K of page i+1 is requested as soon
  // as the score MFMAs have consumed K of page i, and each pair of V rows of
  // page i+1 as soon as P.V has consumed that pair of page i, so each load
  // overlaps the rest of the page's work.
  u32x4_t kr[8];
  u32x2_t vr[kPage];
  int64_t phys_next = 0;
  // Page loads are buffer loads off a per-page resource: one lane-offset
  // register per operand and the row/column steps in the scalar offset.
  const uint32_t k_voff = uint32_t(n16 * a.kc_s + g4 * 8) * 2u;
  const uint32_t v_voff = uint32_t(lane) * 8u;
  const int v_row_bytes = int(a.vc_s) * 2;
  auto issue_k = [&](int i) {
    phys_next = bt_ahead;
    if (i + 1 < npw) bt_ahead = bt_s[p0 + wave + (i + 1) * kW];
    const __amdgpu_buffer_rsrc_t rk = page_rsrc(kh + phys_next * a.kc_p);
#pragma unroll
    for (int e = 0; e < 8; ++e) kr[e] = __builtin_amdgcn_raw_buffer_load_b128(rk, k_voff, 64 * e, 0);
  };
  auto issue_v = [&](int i) {
    const __amdgpu_buffer_rsrc_t rv = page_rsrc(vh + phys_next * a.vc_p);
#pragma unroll
    for (int e = 0; e < kPage; ++e)
      vr[e] = __builtin_amdgcn_raw_buffer_load_b64(rv, v_voff, v_row_bytes * e, 0);
  };
  auto issue_v_pair = [&](int j) {  // rows 2j, 2j+1 of the next page
    const __amdgpu_buffer_rsrc_t rv = page_rsrc(vh + phys_next * a.vc_p);
    vr[2 * j] = __builtin_amdgcn_raw_buffer_load_b64(rv, v_voff, v_row_bytes * (2 * j), 0);
    vr[2 * j + 1] = __builtin_amdgcn_raw_buffer_load_b64(rv, v_voff, v_row_bytes * (2 * j + 1), 0);
  };

  // Fused step: the new token's K and V rows come from k_new / v_new (the
  // cached row at that slot is stale until the append lands).  The wave that
  // owns the new token's page (always its final page) scores the new key with
  // the same 8 MFMAs as a page (each MFMA output element depends only on its
  // own row and column, so the value is the one the page pass would produce
  // from the cache) and substitutes v_new for that V row; it also writes the
  // append.  In the attention block the key first needs its RMSNorm and RoPE:
  // there the workgroup's last wave, idle while the q rows are staged,
  // prepares both rows in LDS and writes the append.
  const bool has_new = kFused && p0 <= last_page && last_page < p1;  // uniform
  auto stage_new = [&] {
    const int c = (lane & 31) * 8;
    u32x4_t krow = {0u, 0u, 0u, 0u};
    if constexpr (kProlog) {
      // RMSNorm + partial RoPE of the raw key row (both 32-lane halves compute it)
      const u32x4_t xw = ld16(knrow + c);
      const u32x4_t ww = ld16(a.kw + c);
      // chunk l (dims 8l..8l+7) pairs with chunk l +- half/8
      const int hc = a.rope_dim / 16, l32 = lane & 31;
      const bool first = l32 < hc, second = l32 >= hc && l32 < 2 * hc;
      const int partner = (lane & 32) | (first ? l32 + hc : second ? l32 - hc : l32);
      const float pf = float(seq_len - 1);  // = float(pos[b])
      float sn8[8], cs8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sn8[e] = 0.f;
        cs8[e] = 1.f;
        if (first || second)
          rope_sincos(pf, a.inv_freq[(first ? c : c - 8 * hc) + e], sn8[e], cs8[e]);
      }
      const float rs = rms_rsigma(rms_acc8(xw, 0.f), kD, a.eps);
      float y[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        y[2 * e] = round_bf16(rms_apply(bf16_lo(xw[e]), rs, bf16_lo(ww[e])));
        y[2 * e + 1] = round_bf16(rms_apply(bf16_hi(xw[e]), rs, bf16_hi(ww[e])));
      }
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float o[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const float other = __shfl(y[e + u], partner);
          o[u] = y[e + u];
          if (first || second) {
            float o1, o2;
            if (first) {
              rope_rotate(y[e + u], other, cs8[e + u], sn8[e + u], o1, o2);
              o[u] = o1;
            } else {
              rope_rotate(other, y[e + u], cs8[e + u], sn8[e + u], o1, o2);
              o[u] = o2;
            }
          }
        }
        krow[e / 2] = pack_bf16x2(o[0], o[1]);
      }
    }
    const int64_t phys = btrow[last_page];
    if (lane < 32) {
      st16(&sm.kn[c], krow);
      st16(a.kc + phys * a.kc_p + h * a.kc_h + last_slot * a.kc_s + c, krow);
    } else {
      const u32x4_t vrow = ld16(vnrow + c);
      st16(&sm.vn[c], vrow);
      st16(a.vc + phys * a.vc_p + h * a.vc_h + last_slot * a.vc_s + c, vrow);
    }
  };

  // The group's 4 query rows, staged once in LDS; each page rebuilds the MFMA
  // A operand from it (rows 4..15 of the operand are zero).
  if constexpr (kProlog) {
    if (has_new && wave == kW - 1) stage_new();
    // The RoPE inputs are fetched with the rows: lane i later rotates pair
    // (head i / half, j = i % half).
    const int half = a.rope_dim / 2;
    const float pf = float(seq_len - 1);  // = float(pos[b])
    float sn = 0.f, cs = 1.f;
    if (threadIdx.x < kG * half) rope_sincos(pf, a.inv_freq[threadIdx.x % half], sn, cs);
    // RMSNorm: 32 lanes per row, 8 elements each (rms_rsigma's layout).
    if (threadIdx.x < kG * kD / 8) {
      const int r = threadIdx.x >> 5, c = (threadIdx.x & 31) * 8;
      const u32x4_t xw = q_pre;  // q row r, dims c..c+7 (r == r_q, c == c_q)
      const u32x4_t ww = ld16(a.qw + c);
      const float ss = rms_acc8(xw, 0.f);
      const float rs = rms_rsigma(ss, kD, a.eps);
      u32x4_t y;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        y[e] = pack_bf16x2(rms_apply(bf16_lo(xw[e]), rs, bf16_lo(ww[e])),
                           rms_apply(bf16_hi(xw[e]), rs, bf16_hi(ww[e])));
      st16(&sm_q[r][c], y);
    }
    __syncthreads();
    // partial RoPE on dims [0, rope_dim): one lane per (head, pair)
    if (threadIdx.x < kG * half) {  // rope_dim <= 128: one pass covers every pair
      const int i = threadIdx.x, r = i / half, j = i - r * half;
      float o1, o2;
      rope_rotate(bf16_to_f32(sm_q[r][j]), bf16_to_f32(sm_q[r][j + half]), cs, sn, o1, o2);
      const uint32_t pk = pack_bf16x2(o1, o2);
      sm_q[r][j] = bf16_t(pk & 0xffffu);
      sm_q[r][j + half] = bf16_t(pk >> 16);
    }
  } else if (threadIdx.x < kG * kD / 8) {
    const int r = threadIdx.x >> 5, c = (threadIdx.x & 31) * 8;
    const bf16_t *qrow = a.q + b * a.qs_b + (h * kG + r) * a.qs_h;
    u32x4_t w;
    if (q_fast) {
      w = q_pre;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = uint32_t(qrow[(c + 2 * e) * a.qs_d]) |
               (uint32_t(qrow[(c + 2 * e + 1) * a.qs_d]) << 16);
    }
    st16(&sm_q[r][c], w);
  }
  __syncthreads();

  WY_DSTAMP(2);
  f32x4_t sc_new = {0.f, 0.f, 0.f, 0.f};
  u32x2_t vnew = {0u, 0u};
  bool owns_new = false;
  if constexpr (kFused) {
    owns_new = has_new && (last_page - p0) % kW == wave;
    if (owns_new) {
      // the attention block staged both rows in LDS; the plain step reads
      // k_new / v_new here and writes the append itself
      const bf16_t *ksrc = kProlog ? sm.kn : knrow;
      u32x4_t kn[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) kn[e] = ld16(ksrc + g4 * 8 + 32 * e);
      vnew = *reinterpret_cast<const u32x2_t *>((kProlog ? sm.vn : vnrow) + lane * 4);
      if constexpr (!kProlog) {
        const int64_t phys = btrow[last_page];
        const int c = (lane & 31) * 8;
        if (lane < 32)
          st16(a.kc + phys * a.kc_p + h * a.kc_h + last_slot * a.kc_s + c, ld16(knrow + c));
        else
          st16(a.vc + phys * a.vc_p + h * a.vc_h + last_slot * a.vc_s + c, ld16(vnrow + c));
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const u32x4_t qw = n16 < kG ? ld16(&sm_q[n16 & 3][32 * e + 8 * g4])
                                    : u32x4_t{0u, 0u, 0u, 0u};
        sc_new = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, qw),
                                                         __builtin_bit_cast(bf16x8_t, kn[e]),
                                                         sc_new, 0, 0, 0);
      }
    }
  }

  if (npw > 0) {
    issue_k(0);
    issue_v(0);
  }

  // One page of work; kMore: the wave has a next page whose loads to issue.
  auto page = [&](int i, auto more) {
    constexpr bool kMore = decltype(more)::value;
    const int p = p0 + wave + i * kW;
    const bool new_page = kFused && !kMore && owns_new;  // then p == last_page

    // ---- scores: 4 heads x 16 tokens in lanes 0..15 ------------------------
    f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
    // q is re-read from LDS for every page (the opaque offset keeps the
    // compiler from hoisting 32 loop-invariant registers out of the loop).
    uint32_t q_off = uint32_t(((n16 & 3) * (kD + 8) + 8 * g4) * 2);
    asm volatile("" : "+v"(q_off));
    const char *q_lds = reinterpret_cast<const char *>(&sm_q[0][0]) + q_off;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const u32x4_t qw = n16 < kG ? ld16(q_lds + 64 * e) : u32x4_t{0u, 0u, 0u, 0u};
      sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, qw),
                                                   __builtin_bit_cast(bf16x8_t, kr[e]), sc,
                                                   0, 0, 0);
    }
    if constexpr (kMore) issue_k(i + 1);
    if (new_page && n16 == last_slot) sc = sc_new;

    const int valid_rows = seq_len - p * kPage;  // >= 1
    const bool valid = n16 < valid_rows;
    float pr[kG], alpha[kG];
#pragma unroll
    for (int r = 0; r < kG; ++r) {
      const float x = valid ? sc[r] * a.scale : -INFINITY;
      const float mx = readlane0(max16(x));
      const float m_new = fmaxf(m_run[r], mx);
      alpha[r] = __expf(m_run[r] - m_new);
      pr[r] = __expf(x - m_new);
      const float ps = readlane0(sum16(pr[r]));
      l_run[r] = l_run[r] * alpha[r] + ps;
      m_run[r] = m_new;
    }
    {
      // even token lanes pair their P with the next token's (lane swap)
      u32x4_t w;
#pragma unroll
      for (int r = 0; r < kG; ++r) w[r] = pack_bf16x2(pr[r], __shfl_xor(pr[r], 1));
      if (lane < kPage && (lane & 1) == 0) sm_p[wave][lane >> 1] = w;
    }
    __builtin_amdgcn_wave_barrier();

    // Rows past the sequence end may hold anything (even NaN): zero them so
    // 0 * garbage cannot reach the accumulator.
    if (valid_rows < kPage) {
#pragma unroll
      for (int e = 0; e < kPage; ++e)
        if (e >= valid_rows) vr[e] = u32x2_t{0u, 0u};
    }
    // ---- acc = acc * alpha + P V (lane: dims 4*lane..+3, all 16 tokens) ----------
#pragma unroll
    for (int r = 0; r < kG; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[r][e] *= alpha[r];
    // Token pairs (2j, 2j+1): P pairs come from LDS, V pairs per dim are
    // assembled with v_perm_b32, and each (head, dim, pair) is one
    // v_dot2_f32_bf16 (bf16 products summed in fp32).
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int j = 0; j < kPage / 2; ++j) {
      const u32x4_t pp = sm_p[wave][j];
      u32x2_t va = vr[2 * j], vb = vr[2 * j + 1];
      if constexpr (kFused && !kMore) {
        if (new_page && 2 * j == last_slot) va = vnew;
        if (new_page && 2 * j + 1 == last_slot) vb = vnew;
      }
      const uint32_t vd[4] = {__builtin_amdgcn_perm(vb[0], va[0], 0x05040100u),
                              __builtin_amdgcn_perm(vb[0], va[0], 0x07060302u),
                              __builtin_amdgcn_perm(vb[1], va[1], 0x05040100u),
                              __builtin_amdgcn_perm(vb[1], va[1], 0x07060302u)};
#pragma unroll
      for (int r = 0; r < kG; ++r) {
        // copy the lane out first: bit-casting an ext-vector element directly
        // is lowered as a cast of element 0
        const uint32_t pr_pair = pp[r];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[r][e] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pr_pair),
                                                      __builtin_bit_cast(bf16x2_t, vd[e]),
                                                      acc[r][e], false);
      }
      if constexpr (kMore) issue_v_pair(j);
    }
    __builtin_amdgcn_wave_barrier();
  };
  if (npw > 0) {
    for (int i = 0; i + 1 < npw; ++i) page(i, std::true_type{});
    page(npw - 1, std::false_type{});
  }

  WY_DSTAMP(3);
  // ---- merge the four wave states through LDS ---------------------------------
#pragma unroll
  for (int r = 0; r < kG; ++r)
    sm_acc[wave][r][lane] = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < kG; ++r) {
      sm_ml[wave][0][r] = m_run[r];
      sm_ml[wave][1][r] = l_run[r];
    }
  }
  __syncthreads();

  WY_DSTAMP(4);
  // waves 0..3 finish one query head each
  const int r = wave & (kG - 1);
  const bool head_wave = wave < kG;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kW; ++w) M = fmaxf(M, sm_ml[w][0][r]);
  float L = 0.f;
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  if (head_wave) {
#pragma unroll 4
    for (int w = 0; w < kW; ++w) {
      const float e = __expf(sm_ml[w][0][r] - M);
      L += e * sm_ml[w][1][r];
      const float4 x = sm_acc[w][r][lane];
      A.x += e * x.x;
      A.y += e * x.y;
      A.z += e * x.z;
      A.w += e * x.w;
    }
  }
  const int hq = h * kG + r;
  if constexpr (kFused) {
    if (nact == 1) {  // the only split: finish here, no scratch round trip
      if (head_wave) store_out4(a, b, hq, lane * 4, A, L, &gate_pre);
      return;
    }
  }
  float *adst = a.ap + b * a.a_b + hq * a.a_h + s * a.a_s + lane * 4;
  float *mdst = a.mp + b * a.ml_b + hq * a.ml_h + s * a.ml_s;
  float *ldst = a.lp + b * a.ml_b + hq * a.ml_h + s * a.ml_s;
  if constexpr (!kFused) {
    if (head_wave) {
      *reinterpret_cast<float4 *>(adst) = A;
      if (lane == 0) {
        *mdst = M;
        *ldst = L;
      }
    }
  } else {
    // Publish this split with device-coherent stores, wait until they have
    // completed, then count it.  The workgroup that completes the count
    // merges, reading the partials coherently.  (A workgroup-scope release
    // fence alone does not wait for the stores to complete on gfx950, hence
    // the explicit vmcnt wait before the barrier.)  With more than
    // kMergeGroup splits the count is per group of kMergeGroup splits, whose
    // last workgroup publishes the group's merged state in the group's first
    // slot and counts it on the (b, h) counter.
    auto publish = [&](float *ad, float *md, float *ldp, float4 Av, float Mv, float Lv) {
      if (head_wave) {
        st_coherent4(ad, Av);
        if (lane == 0) {
          st_coherent(md, Mv);
          st_coherent(ldp, Lv);
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __syncthreads();
    };
    auto count = [&](int *cnt, int need) {
      if (threadIdx.x == 0) {
        const int done = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
        const int last = done == need - 1;
        if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sm.last = last;
      }
      __syncthreads();
      return sm.last != 0;
    };
    publish(adst, mdst, ldst, A, M, L);
    WY_DSTAMP(5);
    int *top = a.counters + b * a.hkv + h;
    const int ng = a.two_level ? (nact + kMergeGroup - 1) / kMergeGroup : 1;
    if (ng == 1) {
      const bool lastc = count(top, nact);
      WY_DSTAMP(6);
#if WY_TRACE
      if (threadIdx.x == 0 && blockIdx.x < 1024) {
        unsigned xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        g_dtrace[blockIdx.x * 16 + 12] = (unsigned long long)b | ((unsigned long long)h << 8) |
                                         ((unsigned long long)s << 16) |
                                         ((unsigned long long)nact << 24) |
                                         ((unsigned long long)(p1 - p0) << 32) |
                                         ((unsigned long long)lastc << 48) |
                                         ((unsigned long long)(xcc & 15) << 52);
      }
#endif
      if (!lastc || !head_wave) return;
      const Merged mr = merge_slots<true>(a, b, hq, 0, 1, nact, lane);
      WY_DSTAMP(7);
      store_out4(a, b, hq, lane * 4, mr.A, mr.L, &gate_pre);
#if WY_TRACE
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      WY_DSTAMP(8);
#endif
      return;
    }
    const int g = s / kMergeGroup;
    const int g0 = g * kMergeGroup;
    int *gcnt = a.counters + a.batch * a.hkv + (b * a.hkv + h) * (kMaxSplits / kMergeGroup) + g;
    if (!count(gcnt, min(kMergeGroup, nact - g0))) return;
    Merged gm = {0.f, 0.f, make_float4(0.f, 0.f, 0.f, 0.f)};
    if (head_wave) gm = merge_slots<true>(a, b, hq, g0, 1, min(kMergeGroup, nact - g0), lane);
    float *gslot_a = a.ap + b * a.a_b + hq * a.a_h + g0 * a.a_s + lane * 4;
    float *gslot_m = a.mp + b * a.ml_b + hq * a.ml_h + g0 * a.ml_s;
    float *gslot_l = a.lp + b * a.ml_b + hq * a.ml_h + g0 * a.ml_s;
    publish(gslot_a, gslot_m, gslot_l, gm.A, gm.M, gm.L);
    if (!count(top, ng) || !head_wave) return;
    const Merged mr = merge_slots<true>(a, b, hq, 0, kMergeGroup, ng, lane);
    store_out4(a, b, hq, lane * 4, mr.A, mr.L, &gate_pre);
  }
}

// One wavefront per (sequence, query head).
__global__ __launch_bounds__(64) void paged_decode_combine_kernel(const DecodeArgs a) {
  const int b = blockIdx.x, hq = blockIdx.y;
  const int seq_len = int(a.pos[b]) + 1;
  const int npg = (seq_len + kPage - 1) / kPage;
  const int pps = split_pps(npg, a.min_pps);
  const Merged mr = merge_all<false>(a, b, hq, (npg + pps - 1) / pps, threadIdx.x);
  store_out4(a, b, hq, threadIdx.x * 4, mr.A, mr.L);
}

bool cache_layout_ok(const void *kc, const void *vc, const int64_t *kcs, const int64_t *vcs) {
  return kcs[3] == 1 && vcs[3] == 1 && kcs[2] % 8 == 0 && vcs[2] % 8 == 0 &&
         kcs[1] % 8 == 0 && vcs[1] % 8 == 0 && kcs[0] % 8 == 0 && vcs[0] % 8 == 0 &&
         wyh::aligned16(kc) && wyh::aligned16(vc);
}

bool scratch_layout_ok(const void *acc, const int64_t *as) {
  return as[3] == 1 && as[2] % 4 == 0 && as[1] % 4 == 0 && as[0] % 4 == 0 &&
         wyh::aligned16(acc);
}

bool q_layout_ok(const void *q, const int64_t *qs) {
  return qs[2] != 1 || (qs[0] % 8 == 0 && qs[1] % 8 == 0 && wyh::aligned16(q));
}

bool out_layout_ok(const void *out, const int64_t *os) {
  return os[2] != 1 || (os[0] % 4 == 0 && os[1] % 4 == 0 &&
                        (reinterpret_cast<uintptr_t>(out) & 7u) == 0);
}

// Target item count of the one-launch step's balanced order: one per CU.
// A batch whose splits at the caller's floor would exceed it gets longer
// splits (64 x 32k tokens: 1024 pages each, 256 items), while a batch with
// one very long sequence among short ones keeps the short floor and cuts the
// long sequence into many splits.  Measured over 256/512/1024/2048/4096 on
// B = 1..64 x 32k tokens: fewer, longer splits stream faster at every batch
// (64 x 32k: 741 us at 256, 766 us at 2048), and short batches never reach
// the target, so they are unchanged.
#ifndef WY_DECODE_WORK_ITEMS
#define WY_DECODE_WORK_ITEMS 256
#endif
constexpr int kWorkItems = WY_DECODE_WORK_ITEMS;
constexpr int kLongTablePages = 1024;

int split_grid_z(int max_pages, int min_pps) {
  const int z = (max_pages + min_pps - 1) / min_pps;
  return z > kMaxSplits ? kMaxSplits : z;
}

template <bool kFused, int kW, bool kProlog = false>
int launch_split_w(dim3 grid, const DecodeArgs &a, hipStream_t st) {
  const size_t lds = sizeof(SplitLds<kW>);
  auto *fn = paged_decode_split_kernel<kFused, kW, kProlog>;
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(fn),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             int(lds));
    if (e != hipSuccess) return int(e);
  }
  fn<<<grid, 64 * kW, lds, st>>>(a);
  return wyh::launch_status();
}

template <bool kFused, bool kProlog = false>
int launch_split(const DecodeArgs &args, int batch, int num_kv_heads, int max_pages, int min_pps,
                 void *stream) {
  DecodeArgs a = args;
  a.batch = batch;
  a.bt_cols = max_pages;
  // The balanced order for mid-size batches, and for the one-launch step of
  // small batches over long tables; small batches over short tables keep the
  // direct order, which needs no pass over pos before the first loads.
  a.balanced = batch <= 64 * kBalancedChunks &&
               (batch >= kBalancedMinBatch || (kFused && max_pages >= kLongTablePages));
  a.two_level = 1;
  int64_t items = int64_t(batch) * num_kv_heads * split_grid_z(max_pages, min_pps);
  if (kFused && a.balanced) {
    // The one-launch step merges its own splits, so it may size them from
    // the batch's total length: at most kWorkItems + B*H items.
    a.work_items = kWorkItems;
    items = std::min<int64_t>(items, kWorkItems + int64_t(batch) * num_kv_heads);
  }
  const dim3 grid{unsigned(items)};
  return launch_split_w<kFused, kWaves, kProlog>(grid, a, static_cast<hipStream_t>(stream));
}

DecodeArgs base_args(const void *q, const int64_t *qs, const void *k_cache,
                     const void *v_cache, const int64_t *kcs, const int64_t *vcs,
                     const int32_t *block_table, int64_t bt_stride0, const int64_t *pos,
                     float *m_partial, float *l_partial, float *acc_partial,
                     const int64_t *mls, const int64_t *as, int num_kv_heads, int head_dim,
                     int min_pps) {
  DecodeArgs a = {};
  a.q = static_cast<const bf16_t *>(q);
  a.qs_b = qs[0];
  a.qs_h = qs[1];
  a.qs_d = qs[2];
  a.kc = static_cast<bf16_t *>(const_cast<void *>(k_cache));
  a.vc = static_cast<bf16_t *>(const_cast<void *>(v_cache));
  a.kc_p = kcs[0];
  a.kc_h = kcs[1];
  a.kc_s = kcs[2];
  a.vc_p = vcs[0];
  a.vc_h = vcs[1];
  a.vc_s = vcs[2];
  a.bt = block_table;
  a.bt_b = bt_stride0;
  a.pos = pos;
  a.mp = m_partial;
  a.lp = l_partial;
  a.ap = acc_partial;
  a.ml_b = mls[0];
  a.ml_h = mls[1];
  a.ml_s = mls[2];
  a.a_b = as[0];
  a.a_h = as[1];
  a.a_s = as[2];
  a.scale = 1.0f / sqrtf(float(head_dim));
  a.min_pps = min_pps;
  a.hkv = num_kv_heads;
  return a;
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
  if (!cache_layout_ok(k_cache, v_cache, kcs, vcs) || !scratch_layout_ok(acc_partial, as) ||
      !q_layout_ok(q, qs))
    return WY_E_LAYOUT;
  if (batch == 0) return WY_OK;
  const DecodeArgs a = base_args(q, qs, k_cache, v_cache, kcs, vcs, block_table, bt_stride0,
                                 pos, m_partial, l_partial, acc_partial, mls, as,
                                 num_kv_heads, head_dim, min_pages_per_split);
  return launch_split<false>(a, batch, num_kv_heads, max_pages, min_pages_per_split, stream);
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
  if (!scratch_layout_ok(acc_partial, as) || !out_layout_ok(out, os)) return WY_E_LAYOUT;
  if (batch == 0) return WY_OK;
  DecodeArgs a = {};
  a.mp = const_cast<float *>(m_partial);
  a.lp = const_cast<float *>(l_partial);
  a.ap = const_cast<float *>(acc_partial);
  a.ml_b = mls[0];
  a.ml_h = mls[1];
  a.ml_s = mls[2];
  a.a_b = as[0];
  a.a_h = as[1];
  a.a_s = as[2];
  a.pos = pos;
  a.min_pps = min_pages_per_split;
  a.two_level = 1;
  a.out = static_cast<bf16_t *>(out);
  a.o_b = os[0];
  a.o_h = os[1];
  a.o_d = os[2];
  dim3 grid(batch, num_q_heads);
  paged_decode_combine_kernel<<<grid, 64, 0, static_cast<hipStream_t>(stream)>>>(a);
  return wyh::launch_status();
}

extern "C" int wy_paged_decode_step(const void *q, const int64_t *qs, const void *k_new,
                                    const void *v_new, const int64_t *kns,
                                    const int64_t *vns, void *k_cache, void *v_cache,
                                    const int64_t *kcs, const int64_t *vcs,
                                    const int32_t *block_table, int64_t bt_stride0,
                                    const int64_t *pos, float *m_partial, float *l_partial,
                                    float *acc_partial, const int64_t *mls,
                                    const int64_t *as, int32_t *counters, const void *gate,
                                    const int64_t *gs, void *out, const int64_t *os,
                                    int batch, int num_q_heads, int num_kv_heads,
                                    int head_dim, int max_pages, int min_pages_per_split,
                                    void *stream) {
  if (!q || !qs || !k_new || !v_new || !kns || !vns || !k_cache || !v_cache || !kcs ||
      !vcs || !block_table || !pos || !m_partial || !l_partial || !acc_partial || !mls ||
      !as || !counters || !out || !os || (gate && !gs))
    return WY_E_NULL;
  if (batch < 0 || num_kv_heads <= 0 || max_pages <= 0 || min_pages_per_split <= 0)
    return WY_E_SHAPE;
  if (head_dim != kD || num_q_heads != kG * num_kv_heads) return WY_E_UNSUPPORTED;
  if (!cache_layout_ok(k_cache, v_cache, kcs, vcs) || !scratch_layout_ok(acc_partial, as) ||
      !q_layout_ok(q, qs) || !out_layout_ok(out, os) || kns[2] != 1 || vns[2] != 1 ||
      kns[0] % 8 || kns[1] % 8 || vns[0] % 8 || vns[1] % 8 || !wyh::aligned16(k_new) ||
      !wyh::aligned16(v_new))
    return WY_E_LAYOUT;
  if (batch == 0) return WY_OK;
  DecodeArgs a = base_args(q, qs, k_cache, v_cache, kcs, vcs, block_table, bt_stride0, pos,
                           m_partial, l_partial, acc_partial, mls, as, num_kv_heads,
                           head_dim, min_pages_per_split);
  a.kn = static_cast<const bf16_t *>(k_new);
  a.vn = static_cast<const bf16_t *>(v_new);
  a.kn_b = kns[0];
  a.kn_h = kns[1];
  a.vn_b = vns[0];
  a.vn_h = vns[1];
  a.counters = counters;
  a.gate = static_cast<const bf16_t *>(gate);
  if (gate) {
    a.g_b = gs[0];
    a.g_h = gs[1];
    a.g_d = gs[2];
  }
  a.out = static_cast<bf16_t *>(out);
  a.o_b = os[0];
  a.o_h = os[1];
  a.o_d = os[2];
  return launch_split<true>(a, batch, num_kv_heads, max_pages, min_pages_per_split, stream);
}

extern "C" int wy_paged_decode_block(const void *q_raw, const int64_t *qs, const void *gate,
                                     const int64_t *gs, const void *k_raw, const int64_t *kns,
                                     const void *v_raw, const int64_t *vns,
                                     const void *q_norm_weight, const void *k_norm_weight,
                                     float eps, const float *inv_freq, int rotary_dim,
                                     void *k_cache, void *v_cache, const int64_t *kcs,
                                     const int64_t *vcs, const int32_t *block_table,
                                     int64_t bt_stride0, const int64_t *pos, float *m_partial,
                                     float *l_partial, float *acc_partial, const int64_t *mls,
                                     const int64_t *as, int32_t *counters, void *out,
                                     const int64_t *os, int batch, int num_q_heads,
                                     int num_kv_heads, int head_dim, int max_pages,
                                     int min_pages_per_split, void *stream) {
  if (!q_raw || !qs || !gate || !gs || !k_raw || !kns || !v_raw || !vns || !q_norm_weight ||
      !k_norm_weight || !inv_freq || !k_cache || !v_cache || !kcs || !vcs || !block_table ||
      !pos || !m_partial || !l_partial || !acc_partial || !mls || !as || !counters || !out ||
      !os)
    return WY_E_NULL;
  if (batch < 0 || num_kv_heads <= 0 || max_pages <= 0 || min_pages_per_split <= 0)
    return WY_E_SHAPE;
  if (head_dim != kD || num_q_heads != kG * num_kv_heads) return WY_E_UNSUPPORTED;
  if (rotary_dim < 0 || rotary_dim > 128 || rotary_dim % 16 != 0) return WY_E_UNSUPPORTED;
  if (!cache_layout_ok(k_cache, v_cache, kcs, vcs) || !scratch_layout_ok(acc_partial, as) ||
      !out_layout_ok(out, os) || qs[2] != 1 || qs[0] % 8 || qs[1] % 8 || !wyh::aligned16(q_raw) ||
      kns[2] != 1 || vns[2] != 1 || kns[0] % 8 || kns[1] % 8 || vns[0] % 8 || vns[1] % 8 ||
      !wyh::aligned16(k_raw) || !wyh::aligned16(v_raw) || !wyh::aligned16(q_norm_weight) ||
      !wyh::aligned16(k_norm_weight))
    return WY_E_LAYOUT;
  if (batch == 0) return WY_OK;
  DecodeArgs a = base_args(q_raw, qs, k_cache, v_cache, kcs, vcs, block_table, bt_stride0, pos,
                           m_partial, l_partial, acc_partial, mls, as, num_kv_heads, head_dim,
                           min_pages_per_split);
  a.kn = static_cast<const bf16_t *>(k_raw);
  a.vn = static_cast<const bf16_t *>(v_raw);
  a.kn_b = kns[0];
  a.kn_h = kns[1];
  a.vn_b = vns[0];
  a.vn_h = vns[1];
  a.counters = counters;
  a.gate = static_cast<const bf16_t *>(gate);
  a.g_b = gs[0];
  a.g_h = gs[1];
  a.g_d = gs[2];
  a.out = static_cast<bf16_t *>(out);
  a.o_b = os[0];
  a.o_h = os[1];
  a.o_d = os[2];
  a.qw = static_cast<const bf16_t *>(q_norm_weight);
  a.kw = static_cast<const bf16_t *>(k_norm_weight);
  a.inv_freq = inv_freq;
  a.eps = eps;
  a.rope_dim = rotary_dim;
  return launch_split<true, true>(a, batch, num_kv_heads, max_pages, min_pages_per_split,
                                  stream);
}

// ---- decode step without a caller workspace -----------------------------------
//
// The split partials and merge counters of wy_paged_decode_step live in this
// file-scope device array instead of caller memory: m and l [rows][128] fp32,
// acc [rows][128][256] fp32 and the counters, for rows = batch * num_q_heads <=
// kNoAllocMaxRows (64 MiB + 514 KiB per GPU, held until the process ends).  In
// host code `scratch` only names the symbol: its device address comes from
// hipGetSymbolAddress, once per device, and only that address is passed on.
namespace {
constexpr int kNoAllocMaxRows = 512;
constexpr size_t kNoAllocMlFloats = size_t(kNoAllocMaxRows) * kMaxSplits;
constexpr size_t kNoAllocAccFloats = kNoAllocMlFloats * kD;
constexpr size_t kNoAllocCounters = kNoAllocMaxRows / 4 * 9;  // >= batch * num_kv_heads * 9
constexpr size_t kNoAllocBytes = (2 * kNoAllocMlFloats + kNoAllocAccFloats) * 4 +
                                 kNoAllocCounters * 4;
constexpr int kNoAllocMaxDevices = 64;

__global__ void zero_ints_kernel(int32_t *p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {
std::mutex g_noalloc_mu;
unsigned char *g_noalloc_ptr[kNoAllocMaxDevices];

// Device address of this device's `scratch`, resolved on the first call; that
// call also clears the counters on `st` (a fill kernel, ordered before the
// step it precedes on the same stream).  The first call must not be under
// graph capture: the symbol lookup would run during the capture and the
// clearing kernel would only be recorded, not run, so it is refused.
int noalloc_scratch(hipStream_t st, unsigned char **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return int(e);
  if (dev < 0 || dev >= kNoAllocMaxDevices) return WY_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess) return int(e);
    if (cs != hipStreamCaptureStatusNone) return WY_E_UNSUPPORTED;
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return int(e);
    if (!p) return int(hipErrorInvalidSymbol);
    int32_t *cnt = reinterpret_cast<int32_t *>(static_cast<unsigned char *>(p) +
                                               (2 * kNoAllocMlFloats + kNoAllocAccFloats) * 4);
    zero_ints_kernel<<<(int(kNoAllocCounters) + 255) / 256, 256, 0, st>>>(
        cnt, int(kNoAllocCounters));
    e = hipGetLastError();
    if (e != hipSuccess) return int(e);
    g_noalloc_ptr[dev] = static_cast<unsigned char *>(p);
  }
  *out = g_noalloc_ptr[dev];
  return WY_OK;
}
}  // namespace

extern "C" int64_t wy_paged_decode_step_noalloc_max_rows(void) { return kNoAllocMaxRows; }

extern "C" int wy_paged_decode_step_noalloc(const void *q, const int64_t *qs, const void *k_new,
                                            const void *v_new, const int64_t *kns,
                                            const int64_t *vns, void *k_cache, void *v_cache,
                                            const int64_t *kcs, const int64_t *vcs,
                                            const int32_t *block_table, int64_t bt_stride0,
                                            const int64_t *pos, const void *gate,
                                            const int64_t *gs, void *out, const int64_t *os,
                                            int batch, int num_q_heads, int num_kv_heads,
                                            int head_dim, int max_pages,
                                            int min_pages_per_split, void *stream) {
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0) return WY_E_SHAPE;
  if (int64_t(batch) * num_q_heads > kNoAllocMaxRows) return WY_E_CAPACITY;
  if (head_dim != kD || num_q_heads != kG * num_kv_heads) return WY_E_UNSUPPORTED;
  if (batch == 0) return WY_OK;
  unsigned char *base = nullptr;
  const int rc = noalloc_scratch(static_cast<hipStream_t>(stream), &base);
  if (rc != WY_OK) return rc;
  float *m = reinterpret_cast<float *>(base);
  float *l = m + kNoAllocMlFloats;
  float *acc = l + kNoAllocMlFloats;
  int32_t *cnt = reinterpret_cast<int32_t *>(acc + kNoAllocAccFloats);
  // packed [batch, num_q_heads, 128(, 256)] views of the array
  const int64_t mls[3] = {int64_t(num_q_heads) * kMaxSplits, kMaxSplits, 1};
  const int64_t as[4] = {int64_t(num_q_heads) * kMaxSplits * kD, int64_t(kMaxSplits) * kD, kD, 1};
  return wy_paged_decode_step(q, qs, k_new, v_new, kns, vns, k_cache, v_cache, kcs, vcs,
                              block_table, bt_stride0, pos, m, l, acc, mls, as, cnt, gate, gs,
                              out, os, batch, num_q_heads, num_kv_heads, head_dim, max_pages,
                              min_pages_per_split, stream);
}

// ---- streaming floor of the decode step's K/V reads ------------------------------
//
// Reads every K/V page row a decode step attends (pages [0, ceil((pos+1)/16))
// of every sequence and KV head) exactly once, with no attention math.  The
// units (one page of one KV head: 8 KiB of K + 8 KiB of V) are cut into equal
// contiguous ranges over kStreamWaves wavefronts (8 per CU); a wave keeps the
// next unit in flight while it sums the current one.  sums[w] = fp32 sum of
// every element wave w read.  Its time is the HBM floor of the step's access
// pattern with perfect balance: what the decode kernel is measured against.
namespace {
constexpr int kStreamWaves = 2048;
constexpr int kMaxSegsStream = 1024;  // batch * H_kv

__global__ __launch_bounds__(256) void page_stream_kernel(
    const bf16_t *__restrict__ kc, const bf16_t *__restrict__ vc, int64_t kc_p, int64_t kc_h,
    int64_t vc_p, int64_t vc_h, const int32_t *__restrict__ bt, int64_t bt_b,
    const int64_t *__restrict__ pos, int batch, int hkv, float *__restrict__ sums) {
  __shared__ int prefix[kMaxSegsStream + 1];
  const int lane = threadIdx.x & 63;
  const int nseg = batch * hkv;
  if (threadIdx.x < 64) {  // segment prefix sums, 64 segments per pass
    int carry = 0;
    if (lane == 0) prefix[0] = 0;
    for (int c0 = 0; c0 < nseg; c0 += 64) {
      const int sg = c0 + lane;
      int x = sg < nseg ? (int(pos[sg / hkv]) + kPage) / kPage : 0;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
      }
      if (sg < nseg) prefix[sg + 1] = carry + x;
      carry += __shfl(x, 63);
    }
  }
  __syncthreads();
  const int units = prefix[nseg];
  const int gw = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int u0 = int(int64_t(gw) * units / kStreamWaves);
  const int u1 = int(int64_t(gw + 1) * units / kStreamWaves);
  int seg = 0;
  {
    int lo = 0, hi = nseg - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (prefix[mid] <= u0) lo = mid;
      else hi = mid - 1;
    }
    seg = lo;
  }
  // seg, u and the page are the same in every lane; stating it
  // (readfirstlane) puts the page's buffer resource in SGPRs, which a buffer
  // load needs (else each load runs in a loop over the distinct values)
  seg = __builtin_amdgcn_readfirstlane(seg);
  auto phys_of = [&](int u) -> int64_t {  // advances seg monotonically
    while (u >= prefix[seg + 1]) ++seg;
    seg = __builtin_amdgcn_readfirstlane(seg);
    const int first = __builtin_amdgcn_readfirstlane(prefix[seg]);
    const int b = seg / hkv;
    // a uniform address read through the constant address space: a scalar
    // load, which a wait on the page loads' vector-memory counter does not cover
    typedef const __attribute__((address_space(4))) int32_t cint_t;
    return int64_t(__builtin_amdgcn_readfirstlane(
        ((cint_t *)bt)[b * bt_b + (u - first)]));
  };
  u32x4_t buf[2][16];
  auto issue = [&](int d, int u) {
    const int64_t phys = phys_of(u);
    const int hh = seg % hkv;
    const __amdgpu_buffer_rsrc_t rk = page_rsrc(kc + phys * kc_p + hh * kc_h);
    const __amdgpu_buffer_rsrc_t rv = page_rsrc(vc + phys * vc_p + hh * vc_h);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      buf[d][e] = __builtin_amdgcn_raw_buffer_load_b128(rk, lane * 16, 1024 * e, 0);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      buf[d][8 + e] = __builtin_amdgcn_raw_buffer_load_b128(rv, lane * 16, 1024 * e, 0);
  };
  float part[4] = {0.f, 0.f, 0.f, 0.f};  // independent sums: no long add chain
  auto consume = [&](int d) {
#pragma unroll
    for (int e = 0; e < 16; ++e)
#pragma unroll
      for (int w = 0; w < 4; ++w) part[w] += bf16_lo(buf[d][e][w]) + bf16_hi(buf[d][e][w]);
  };
  // The main loop issues every load unconditionally, so the wait before
  // consuming one unit leaves the next unit's 16 loads in flight (a load
  // that only some paths issue makes the compiler wait for everything).
  int u = u0;
  if (u0 < u1) issue(0, u0);
  for (; u + 2 < u1; u += 2) {
    issue(1, u + 1);
    consume(0);
    issue(0, u + 2);
    consume(1);
  }
  if (u + 1 < u1) {
    issue(1, u + 1);
    consume(0);
    consume(1);
  } else if (u < u1) {
    consume(0);
  }
  float acc = (part[0] + part[1]) + (part[2] + part[3]);
  acc = wave_sum(acc);
  if (lane == 0) sums[gw] = acc;
}
}  // namespace

extern "C" int64_t wy_page_stream_read_waves(void) { return kStreamWaves; }

extern "C" int wy_page_stream_read(const void *k_cache, const void *v_cache,
                                   const int64_t *kcs, const int64_t *vcs,
                                   const int32_t *block_table, int64_t bt_stride0,
                                   const int64_t *pos, int batch, int num_kv_heads,
                                   int head_dim, float *sums, void *stream) {
  if (!k_cache || !v_cache || !kcs || !vcs || !block_table || !pos || !sums) return WY_E_NULL;
  if (batch < 0 || num_kv_heads <= 0) return WY_E_SHAPE;
  if (head_dim != kD || batch * num_kv_heads > kMaxSegsStream) return WY_E_UNSUPPORTED;
  // whole 512-byte rows, 16 rows per page: the loads address row e of a page as 1024 e
  if (!cache_layout_ok(k_cache, v_cache, kcs, vcs) || kcs[2] != kD || vcs[2] != kD)
    return WY_E_LAYOUT;
  if (batch == 0) return WY_OK;
  page_stream_kernel<<<kStreamWaves / 4, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const bf16_t *>(k_cache), static_cast<const bf16_t *>(v_cache), kcs[0], kcs[1],
      vcs[0], vcs[1], block_table, bt_stride0, pos, batch, num_kv_heads, sums);
  return wyh::launch_status();
}

#if WY_TRACE
extern "C" int wy_decode_trace_read(void *host, size_t bytes, int clear) {
  if (clear) {
    static unsigned long long zeros[1024 * 16];
    return int(hipMemcpyToSymbol(HIP_SYMBOL(g_dtrace), zeros, sizeof(zeros)));
  }
  return int(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dtrace),
                                 bytes < sizeof(g_dtrace) ? bytes : sizeof(g_dtrace)));
}
#endif
