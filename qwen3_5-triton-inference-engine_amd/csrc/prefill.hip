// Packed varlen causal GQA prefill attention on bf16 MFMA (gfx950): launch
// selection and the C ABI.  The kernel template is in prefill_kernel.h; its
// one-workgroup-per-block variants are instantiated in prefill_direct.hip.
#include "prefill_kernel.h"

using namespace wy_prefill;

namespace wy_prefill {
extern template __global__ void varlen_causal_prefill_kernel<false, 0>(
    const bf16_t *__restrict__ q, int64_t qs_t, int64_t qs_h,
    const bf16_t *__restrict__ k, int64_t ks_t, int64_t ks_h,
    const bf16_t *__restrict__ v, int64_t vs_t, int64_t vs_h, bf16_t *__restrict__ out,
    int64_t os_t,
    int64_t os_h, const int32_t *__restrict__ cu, float qk_scale_log2, int n_seq,
    int n_kv_heads, int n_qblocks, int32_t *__restrict__ counters, const BlockArgs blk,
    int ticket_order);
extern template __global__ void varlen_causal_prefill_kernel<false, 64>(
    const bf16_t *__restrict__ q, int64_t qs_t, int64_t qs_h,
    const bf16_t *__restrict__ k, int64_t ks_t, int64_t ks_h,
    const bf16_t *__restrict__ v, int64_t vs_t, int64_t vs_h, bf16_t *__restrict__ out,
    int64_t os_t,
    int64_t os_h, const int32_t *__restrict__ cu, float qk_scale_log2, int n_seq,
    int n_kv_heads, int n_qblocks, int32_t *__restrict__ counters, const BlockArgs blk,
    int ticket_order);
template <int kRot>
__global__ void short_prefill_kernel(
    const bf16_t *__restrict__ q, int64_t qs_t, int64_t qs_h, const bf16_t *__restrict__ k,
    int64_t ks_t, int64_t ks_h, const bf16_t *__restrict__ v, int64_t vs_t, int64_t vs_h,
    bf16_t *__restrict__ out, int64_t os_t, int64_t os_h, const int32_t *__restrict__ cu,
    float qk_scale_log2, int n_seq, int n_kv_heads, int n_qblocks, const BlockArgs blk,
    int ticket_order);
extern template __global__ void short_prefill_kernel<0>(
    const bf16_t *__restrict__, int64_t, int64_t, const bf16_t *__restrict__, int64_t, int64_t,
    const bf16_t *__restrict__, int64_t, int64_t, bf16_t *__restrict__, int64_t, int64_t,
    const int32_t *__restrict__, float, int, int, int, const BlockArgs, int);
extern template __global__ void short_prefill_kernel<64>(
    const bf16_t *__restrict__, int64_t, int64_t, const bf16_t *__restrict__, int64_t, int64_t,
    const bf16_t *__restrict__, int64_t, int64_t, bf16_t *__restrict__, int64_t, int64_t,
    const int32_t *__restrict__, float, int, int, int, const BlockArgs, int);
}  // namespace wy_prefill

namespace {

// Compute units of the current device (cached per device).
int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

// Query blocks of the launch grid: n_qblocks * batch * H_kv.
int64_t prefill_blocks(int batch, int num_kv_heads, int max_seqlen) {
  return int64_t((max_seqlen + kBQ - 1) / kBQ) * batch * num_kv_heads;
}

}  // namespace

extern "C" int64_t wy_varlen_causal_prefill_workspace_bytes(int batch, int num_kv_heads,
                                                            int max_seqlen) {
  if (batch <= 0 || num_kv_heads <= 0 || max_seqlen <= 0) return 0;
  const int64_t n_wg = prefill_blocks(batch, num_kv_heads, max_seqlen);
  const int64_t n_qblocks = (max_seqlen + kBQ - 1) / kBQ;
  const int cus = device_cus();
  // A grid that fits the chip in one round gains nothing from the queue; the
  // ticket -> block map must fit its LDS.
  if (cus <= 0 || n_wg <= cus || n_wg > INT32_MAX || 2 * int64_t(batch) + n_qblocks + 2 > kPlanLds) return 0;
  return 2 * int64_t(sizeof(int32_t));
}

namespace {

template <bool kList, int kRot>
int set_prefill_lds() {
  // once per instantiation (thread-safe function-local static initialisation)
  static const hipError_t rc = hipFuncSetAttribute(
      reinterpret_cast<const void *>(&varlen_causal_prefill_kernel<kList, kRot>),
      hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  return rc == hipSuccess ? WY_OK : int(rc);
}

bool prefill_layout_ok(const void *q, const int64_t *qs, const void *k, const int64_t *ks,
                       const void *v, const int64_t *vs, const void *out, const int64_t *os) {
  return !(qs[2] != 1 || ks[2] != 1 || vs[2] != 1 || os[2] != 1 || qs[0] % 8 || qs[1] % 8 ||
           ks[0] % 8 || ks[1] % 8 || vs[0] % 8 || vs[1] % 8 || os[0] % 8 || os[1] % 8 ||
           !wyh::aligned16(q) || !wyh::aligned16(k) || !wyh::aligned16(v) ||
           !wyh::aligned16(out));
}

// Order in which the launches hand out query blocks (see the kernel's
// permute); 0 outside tests.
std::atomic<int> g_ticket_order{0};
// Whether one-round grids of short sequences take the eight-wave kernel
// (prefill_short.hip); 1 outside tests.
std::atomic<int> g_short_path{1};

template <int kRot>
int set_short_lds() {
  static const hipError_t rc = hipFuncSetAttribute(
      reinterpret_cast<const void *>(&short_prefill_kernel<kRot>),
      hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  return rc == hipSuccess ? WY_OK : int(rc);
}

// Validated arguments -> one launch (direct or queue).
template <int kRot>
int launch_prefill(const void *q, const int64_t *qs, const void *k, const int64_t *ks,
                   const void *v, const int64_t *vs, void *out, const int64_t *os,
                   const int32_t *cu_seqlens, int batch, int num_kv_heads, int head_dim,
                   int max_seqlen, void *workspace, int64_t workspace_bytes,
                   const BlockArgs &blk, hipStream_t s) {
  int rc = set_prefill_lds<false, kRot>();
  if (rc == WY_OK) rc = set_prefill_lds<true, kRot>();
  if (rc != WY_OK) return rc;
  const int n_qblocks = (max_seqlen + kBQ - 1) / kBQ;
  const int64_t n_wg = prefill_blocks(batch, num_kv_heads, max_seqlen);
  if (n_wg > INT32_MAX) return WY_E_SHAPE;
  // per-sequence DMA ranges are 32-bit byte offsets
  if (int64_t(max_seqlen) * ks[0] * 2 >= INT32_MAX || int64_t(max_seqlen) * vs[0] * 2 >= INT32_MAX ||
      int64_t(max_seqlen) * qs[0] * 2 >= INT32_MAX)
    return WY_E_SHAPE;
  if (kRot > 0 && int64_t(max_seqlen) * blk.gs_t * 2 + int64_t(kG) * blk.gs_h * 2 >= INT32_MAX)
    return WY_E_SHAPE;
  // Queue launch when the caller provides the two counters that
  // wy_varlen_causal_prefill_workspace_bytes asks for; otherwise one
  // workgroup per query block.
  const int64_t need = wy_varlen_causal_prefill_workspace_bytes(batch, num_kv_heads, max_seqlen);
  int32_t *counters = nullptr;
  unsigned grid = unsigned(n_wg);
  // The queue launch's output stores run over a buffer range that ends
  // after the block's last row: a row past it must lie beyond the range,
  // i.e. the row stride covers the four heads' spans.
  const bool rows_disjoint = os[0] >= (kG - 1) * os[1] + kD && os[0] * 2 * kBQ < INT32_MAX;
  if (need > 0 && workspace_bytes >= need && rows_disjoint) {
    counters = static_cast<int32_t *>(workspace);
    grid = unsigned(device_cus());
  }
  const int order = g_ticket_order.load(std::memory_order_relaxed);
  // A one-round grid of sequences of at most two KV tiles: the eight-wave
  // kernel (chosen by the shape alone, so an input always takes the same one).
  // (its per-lane V DMA offsets use 24-bit multiplies: V row stride below
  // 2^24 bytes)
  const bool small_strides = vs[0] < (1 << 23);
  if (!counters && max_seqlen <= 2 * kBN && n_wg <= device_cus() && small_strides &&
      g_short_path.load(std::memory_order_relaxed)) {
    rc = set_short_lds<kRot>();
    if (rc != WY_OK) return rc;
    short_prefill_kernel<kRot><<<dim3(grid), 512, kLdsBytes, s>>>(
        static_cast<const bf16_t *>(q), qs[0], qs[1], static_cast<const bf16_t *>(k), ks[0],
        ks[1], static_cast<const bf16_t *>(v), vs[0], vs[1], static_cast<bf16_t *>(out), os[0],
        os[1], cu_seqlens, kLog2e / sqrtf(float(head_dim)), batch, num_kv_heads, n_qblocks, blk,
        order);
    return wyh::launch_status();
  }
  auto *kern = counters ? varlen_causal_prefill_kernel<true, kRot>
                        : varlen_causal_prefill_kernel<false, kRot>;
  kern<<<dim3(grid), 256, kLdsBytes, s>>>(
      static_cast<const bf16_t *>(q), qs[0], qs[1], static_cast<const bf16_t *>(k), ks[0],
      ks[1], static_cast<const bf16_t *>(v), vs[0], vs[1], static_cast<bf16_t *>(out), os[0],
      os[1], cu_seqlens, kLog2e / sqrtf(float(head_dim)), batch, num_kv_heads, n_qblocks,
      counters, blk, order);
  return wyh::launch_status();
}

}  // namespace

#if WY_TRACE
extern "C" int wy_prefill_trace_read(void *host, size_t bytes, int clear) {
  if (clear) {
    static unsigned long long zeros[256 * 64 * 8];
    return int(hipMemcpyToSymbol(HIP_SYMBOL(g_trace), zeros, sizeof(zeros)));
  }
  return int(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace), bytes < sizeof(g_trace) ? bytes : sizeof(g_trace)));
}
#endif
extern "C" void wy_prefill_set_short_path(int enable) {
  g_short_path.store(enable ? 1 : 0, std::memory_order_relaxed);
}
extern "C" void wy_prefill_set_ticket_order(int order) {
  g_ticket_order.store(order >= 0 && order <= 2 ? order : 0, std::memory_order_relaxed);
}

extern "C" int wy_varlen_causal_prefill(const void *q, const int64_t *qs, const void *k,
                                        const int64_t *ks, const void *v,
                                        const int64_t *vs, void *out, const int64_t *os,
                                        const int32_t *cu_seqlens, int batch,
                                        int num_q_heads, int num_kv_heads, int head_dim,
                                        int max_seqlen, int64_t total_tokens, void *workspace,
                                        int64_t workspace_bytes, void *stream) {
  if (!q || !qs || !k || !ks || !v || !vs || !out || !os || !cu_seqlens) return WY_E_NULL;
  if (batch < 0 || num_kv_heads <= 0 || max_seqlen < 0 || total_tokens < 0)
    return WY_E_SHAPE;
  if (head_dim != kD || num_q_heads != kG * num_kv_heads) return WY_E_UNSUPPORTED;
  if (!prefill_layout_ok(q, qs, k, ks, v, vs, out, os)) return WY_E_LAYOUT;
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace) ||
      (reinterpret_cast<uintptr_t>(workspace) & 3u))
    return WY_E_LAYOUT;
  if (batch == 0 || max_seqlen == 0) return WY_OK;
  return launch_prefill<0>(q, qs, k, ks, v, vs, out, os, cu_seqlens, batch, num_kv_heads,
                           head_dim, max_seqlen, workspace, workspace_bytes, BlockArgs{},
                           static_cast<hipStream_t>(stream));
}

extern "C" int wy_prefill_attention_block(
    const void *q, const int64_t *qs, const void *k, const int64_t *ks, const void *v,
    const int64_t *vs, const void *gate, const int64_t *gs, const void *position_ids,
    int64_t pos_stride, int pos_is_int64, const float *inv_freq, int rotary_dim,
    void *k_cache, void *v_cache, const int64_t *kcs, const int64_t *vcs,
    const int32_t *block_table, int64_t bt_stride0, const int32_t *cu_seqlens, int batch,
    int num_q_heads, int num_kv_heads, int head_dim, int max_seqlen, int64_t total_tokens,
    void *k_roped, float *rope_table, void *out, void *workspace, int64_t workspace_bytes,
    void *stream) {
  if (!q || !qs || !k || !ks || !v || !vs || !gate || !gs || !position_ids || !inv_freq ||
      !k_cache || !v_cache || !kcs || !vcs || !block_table || !cu_seqlens || !k_roped || !rope_table ||
      !out)
    return WY_E_NULL;
  if (batch < 0 || num_kv_heads <= 0 || max_seqlen < 0 || total_tokens < 0)
    return WY_E_SHAPE;
  if (head_dim != kD || num_q_heads != kG * num_kv_heads || rotary_dim != 64)
    return WY_E_UNSUPPORTED;
  // k_roped and out are the block's own contiguous buffers: [T, H_kv, D] and
  // [T, H_q * D]
  const int64_t krs[3] = {int64_t(num_kv_heads) * head_dim, head_dim, 1};
  const int64_t os[3] = {int64_t(num_q_heads) * head_dim, head_dim, 1};
  if (!prefill_layout_ok(q, qs, k_roped, krs, v, vs, out, os) || ks[2] != 1 || gs[2] != 1 ||
      gs[0] % 8 || gs[1] % 8 || !wyh::aligned16(gate))
    return WY_E_LAYOUT;
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace) ||
      (reinterpret_cast<uintptr_t>(workspace) & 3u))
    return WY_E_LAYOUT;
  if (batch == 0 || max_seqlen == 0) return WY_OK;
  // 1. RoPE of K, K/V into the pages, roped K packed for the attention
  if (reinterpret_cast<uintptr_t>(rope_table) & 15u) return WY_E_LAYOUT;
  int rc = wy_prefill_kv_rope_fill(k_cache, v_cache, kcs, vcs, k, ks, v, vs, k_roped, krs,
                                   rope_table, block_table, bt_stride0, cu_seqlens, position_ids,
                                   pos_stride, pos_is_int64, inv_freq, rotary_dim, batch,
                                   num_kv_heads, head_dim, max_seqlen, stream);
  if (rc != WY_OK) return rc;
  // 2. attention with q's RoPE at load and the gate in the epilogue
  const BlockArgs blk{static_cast<const bf16_t *>(gate), gs[0], gs[1], position_ids,
                      pos_stride, pos_is_int64, inv_freq, rope_table};
  return launch_prefill<64>(q, qs, k_roped, krs, v, vs, out, os, cu_seqlens, batch,
                            num_kv_heads, head_dim, max_seqlen, workspace, workspace_bytes,
                            blk, static_cast<hipStream_t>(stream));
}
