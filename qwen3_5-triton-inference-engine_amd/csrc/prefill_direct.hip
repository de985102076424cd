// The one-workgroup-per-block (direct launch) variants of the varlen causal
// prefill kernel, in a unit of their own: it is compiled with the MFMA
// accumulators in VGPRs (-mllvm -amdgpu-mfma-vgpr-form), which the direct
// variants run faster with (config 3: 11.33 -> 10.97 us) and the queue
// variants slower.
#include "prefill_kernel.h"

namespace wy_prefill {
template __global__ void varlen_causal_prefill_kernel<false, 0>(
    const bf16_t *__restrict__ q, int64_t qs_t, int64_t qs_h,
    const bf16_t *__restrict__ k, int64_t ks_t, int64_t ks_h,
    const bf16_t *__restrict__ v, int64_t vs_t, int64_t vs_h, bf16_t *__restrict__ out,
    int64_t os_t,
    int64_t os_h, const int32_t *__restrict__ cu, float qk_scale_log2, int n_seq,
    int n_kv_heads, int n_qblocks, int32_t *__restrict__ counters, const BlockArgs blk,
    int ticket_order);
template __global__ void varlen_causal_prefill_kernel<false, 64>(
    const bf16_t *__restrict__ q, int64_t qs_t, int64_t qs_h,
    const bf16_t *__restrict__ k, int64_t ks_t, int64_t ks_h,
    const bf16_t *__restrict__ v, int64_t vs_t, int64_t vs_h, bf16_t *__restrict__ out,
    int64_t os_t,
    int64_t os_h, const int32_t *__restrict__ cu, float qk_scale_log2, int n_seq,
    int n_kv_heads, int n_qblocks, int32_t *__restrict__ counters, const BlockArgs blk,
    int ticket_order);
}  // namespace wy_prefill

#if WY_TRACE
extern "C" int wy_prefill_direct_trace_read(void *host, size_t bytes, int clear) {
  if (clear) {
    static unsigned long long zeros[256 * 64 * 8];
    return int(hipMemcpyToSymbol(HIP_SYMBOL(g_trace), zeros, sizeof(zeros)));
  }
  return int(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace), bytes < sizeof(g_trace) ? bytes : sizeof(g_trace)));
}
#endif
