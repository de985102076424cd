/*
 * wy_attn.h -- C ABI of the MI355X (gfx950) full-attention hot path of the
 * Qwen3.5 inference engine.
 *
 * Every entry point takes plain device pointers, element strides (int64, in
 * elements, not bytes), sizes and a hipStream_t passed as `void *`.  No torch
 * types cross this boundary.  Each call only enqueues work on `stream`; it
 * never synchronises and never allocates, so it may be captured into a HIP
 * graph.  Return value: 0 on success, a negative WY_E_* code for a rejected
 * argument (nothing was launched), or a positive hipError_t from the launch.
 *
 * Tensor conventions (bf16 is raw IEEE bfloat16 bits, uint16_t):
 *   page pool   k_cache / v_cache [num_pages, H_kv, PAGE=16, D] bf16
 *   block_table [B, max_pages] int32, logical page -> physical page
 *   pos         [B] int64, tokens already cached per sequence
 *   cu_seqlens  [B+1] int32, prefix sums of packed sequence lengths
 *
 * Each function names the reference interface it replaces
 * (sujuyu/qwen3_5-triton-inference-engine, file:line).
 */
#ifndef WY_ATTN_H
#define WY_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WY_PAGE_SIZE 16
#define WY_MAX_SPLITS 128

/* Error codes (negative).  Positive values are hipError_t. */
#define WY_OK 0
#define WY_E_NULL (-1)        /* a required pointer is NULL                     */
#define WY_E_SHAPE (-2)       /* a size is out of the supported range           */
#define WY_E_LAYOUT (-3)      /* a stride / alignment the kernel cannot address */
#define WY_E_UNSUPPORTED (-4) /* head_dim / group size without a kernel         */
#define WY_E_CAPACITY (-5)    /* larger than a fixed-capacity entry point holds */

/* Human-readable text for a return code (static storage). */
const char *wy_status_string(int code);

/* Library version and the code-object target it was built for ("gfx950"). */
const char *wy_build_info(void);

/*
 * K/V append for one decode step.
 *   k_cache[bt[b, pos[b]/16], h, pos[b]%16, :] = k_new[b, h, :]   (same for V)
 * kc_strides/vc_strides: 4 strides of the pools; kn_strides/vn_strides: 3
 * strides of k_new/v_new [B, H_kv, D].  Bit-exact copy.
 * Replaces wy_lib::paged_kv_append
 *   (triton_kernels/gqa_attention_decode_paged.py:254-305, kernel :176-250).
 */
int wy_paged_kv_append(void *k_cache, void *v_cache, const int64_t *kc_strides,
                       const int64_t *vc_strides, const void *k_new,
                       const void *v_new, const int64_t *kn_strides,
                       const int64_t *vn_strides, const int32_t *block_table,
                       int64_t bt_stride0, const int64_t *pos, int batch,
                       int num_kv_heads, int head_dim, void *stream);

/*
 * Packed varlen K/V scatter into the page pool (prefill).
 *   for b, t < n_b: k_cache[bt[b, t/16], h, t%16, :] = k[h, cu[b]+t, :]
 * k/v packed [H_kv, total, D] with strides k_strides/v_strides (any order).
 * Slots past a sequence's end and unreferenced pages are left untouched.
 * Replaces wy_lib::paged_kv_fill_varlen
 *   (triton_kernels/gqa_attention_decode_paged.py:492-561, kernel :398-489)
 * and the single-sequence paged_kv_fill (:355-375) with batch = 1.
 */
int wy_paged_kv_fill_varlen(void *k_cache, void *v_cache,
                            const int64_t *kc_strides, const int64_t *vc_strides,
                            const void *k_packed, const void *v_packed,
                            const int64_t *k_strides, const int64_t *v_strides,
                            const int32_t *block_table, int64_t bt_stride0,
                            const int32_t *cu_seqlens, int batch,
                            int num_kv_heads, int head_dim, int max_seqlen,
                            void *stream);

/*
 * Split-K paged GQA decode, partial pass.  For sequence b, KV head h and split
 * s it reduces pages [s*pps, min((s+1)*pps, npg)) of the sequence, with
 * npg = ceil((pos[b]+1)/16) and pps = max(ceil(npg/128), min_pages_per_split),
 * into m_partial/l_partial [B, H_q, 128] and acc_partial [B, H_q, 128, D]
 * (fp32, unnormalised online-softmax state, natural-log base).  Splits at or
 * past the active count are not written.  q [B, H_q, D] bf16, scale 1/sqrt(D).
 * Replaces wy_lib::paged_gqa_attention_decode_split
 *   (triton_kernels/gqa_attention_decode_paged.py:822-891, kernel :624-733).
 */
int wy_paged_decode_split(const void *q, const int64_t *q_strides,
                          const void *k_cache, const void *v_cache,
                          const int64_t *kc_strides, const int64_t *vc_strides,
                          const int32_t *block_table, int64_t bt_stride0,
                          const int64_t *pos, float *m_partial, float *l_partial,
                          float *acc_partial, const int64_t *ml_strides,
                          const int64_t *acc_strides, int batch, int num_q_heads,
                          int num_kv_heads, int head_dim, int max_pages,
                          int min_pages_per_split, void *stream);

/*
 * Split-K merge: out[b, hq, :] = sum_s a_s acc_s / sum_s a_s l_s with
 * a_s = exp(m_s - max m), over the active splits of sequence b (same
 * partition formula as wy_paged_decode_split).  More than 16 splits merge
 * in two levels (each group of 16 splits, then the group states), the order
 * the one-launch step uses, so both give the same bits for the same
 * partition.  out [B, H_q, D] bf16 with strides out_strides.
 * Replaces wy_lib::paged_gqa_attention_decode_combine
 *   (triton_kernels/gqa_attention_decode_paged.py:901-939, kernel :747-817).
 */
int wy_paged_decode_combine(const float *m_partial, const float *l_partial,
                            const float *acc_partial, const int64_t *ml_strides,
                            const int64_t *acc_strides, const int64_t *pos,
                            void *out, const int64_t *out_strides, int batch,
                            int num_q_heads, int head_dim,
                            int min_pages_per_split, void *stream);

/*
 * Whole decode step in one launch: K/V append + split-K partial + merge
 * (+ optional sigmoid gate).  The new token's K/V rows are taken from
 * k_new/v_new [B, H_kv, D] and written to their page by the workgroup that
 * owns that page; the last workgroup of each (b, kv head) to finish merges
 * the splits -- in two levels, through groups of 16 splits, when a sequence
 * has more than 16 -- (counters [B*H_kv*9] int32: B*H_kv per-(b, kv head)
 * counters, then B*H_kv*8 group counters; zero before the first call and
 * left zero by every call).  gate (may be NULL) [B, H_q, D] with strides
 * gate_strides: out = bf16(bf16(ctx) * sigmoid(gate)), the rounding of the
 * reference's combine followed by its gate pack.  out [B, H_q, D] bf16.
 * Partition: that of wy_paged_decode_split, except that for B <= 256 when
 * B >= 16 or max_pages >= 1024 the floor is raised on the device to
 * max(min_pages_per_split, ceil(H_kv * sum_b npg_b / 256)), so a batch holds
 * about 256 work items (one per CU) once its total length calls for it.
 * Concurrent calls sharing one counters/scratch set race.
 * Replaces the sequence paged_kv_append -> paged_gqa_attention_decode_split
 * -> paged_gqa_attention_decode_combine (-> attention_gate_pack) of
 *   call_paged_gqa_attention_decode_triton
 *   (triton_kernels/gqa_attention_decode_paged.py:963-994) and
 *   engine/runner.py:508-517.
 */
int wy_paged_decode_step(const void *q, const int64_t *q_strides, const void *k_new,
                         const void *v_new, const int64_t *kn_strides,
                         const int64_t *vn_strides, void *k_cache, void *v_cache,
                         const int64_t *kc_strides, const int64_t *vc_strides,
                         const int32_t *block_table, int64_t bt_stride0,
                         const int64_t *pos, float *m_partial, float *l_partial,
                         float *acc_partial, const int64_t *ml_strides,
                         const int64_t *acc_strides, int32_t *counters,
                         const void *gate, const int64_t *gate_strides, void *out,
                         const int64_t *out_strides, int batch, int num_q_heads,
                         int num_kv_heads, int head_dim, int max_pages,
                         int min_pages_per_split, void *stream);

/*
 * wy_paged_decode_step without a caller workspace: the split partials and
 * merge counters live in a static device array of the library (64 MiB +
 * 514 KiB on each GPU the library is used on, held until the process ends),
 * so the call allocates nothing and needs no scratch argument.  Same
 * arguments, semantics and results (bit for bit) as wy_paged_decode_step
 * otherwise.  batch * num_q_heads must not exceed
 * wy_paged_decode_step_noalloc_max_rows() (512), else WY_E_CAPACITY and
 * nothing is launched.  The first call on a device resolves the array's
 * address and clears its counters on `stream`; that first call must run
 * eagerly (returns WY_E_UNSUPPORTED, nothing launched, if `stream` is being
 * captured), later calls may be captured into a graph.  All calls on one GPU share
 * the array: calls that may overlap on one GPU (concurrent streams, host
 * threads) race.  No counterpart in the reference; for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid allocation).
 */
int wy_paged_decode_step_noalloc(const void *q, const int64_t *q_strides, const void *k_new,
                                 const void *v_new, const int64_t *kn_strides,
                                 const int64_t *vn_strides, void *k_cache, void *v_cache,
                                 const int64_t *kc_strides, const int64_t *vc_strides,
                                 const int32_t *block_table, int64_t bt_stride0,
                                 const int64_t *pos, const void *gate,
                                 const int64_t *gate_strides, void *out,
                                 const int64_t *out_strides, int batch, int num_q_heads,
                                 int num_kv_heads, int head_dim, int max_pages,
                                 int min_pages_per_split, void *stream);

/* The row capacity (batch * num_q_heads) of wy_paged_decode_step_noalloc. */
int64_t wy_paged_decode_step_noalloc_max_rows(void);

/*
 * Measurement kernel: reads the K and V rows of every page a decode step
 * attends (pages [0, ceil((pos[b]+1)/16)) of every sequence and KV head, each
 * once) with no attention math, the pages cut into equal contiguous ranges
 * over wy_page_stream_read_waves() wavefronts (8 per CU), one page in flight
 * per wave.  sums[w] (fp32, one per wavefront) = the sum of every element
 * wave w read.  Its duration is the HBM floor of the decode step's access
 * pattern at perfect balance, the practical roofline the decode kernel is
 * measured against.  Pools as wy_paged_decode_step with 512-byte rows
 * (head_dim 256, unit stride).  No counterpart in the reference (a
 * measurement of this build).
 */
int wy_page_stream_read(const void *k_cache, const void *v_cache, const int64_t *kc_strides,
                        const int64_t *vc_strides, const int32_t *block_table,
                        int64_t bt_stride0, const int64_t *pos, int batch, int num_kv_heads,
                        int head_dim, float *sums, void *stream);

/* Wavefronts (= entries of `sums`) of wy_page_stream_read. */
int64_t wy_page_stream_read_waves(void);

/*
 * Packed varlen causal GQA prefill attention on bf16 MFMA.
 *   out[t, hq, :] = softmax_{j<=i}(q_i . k_j / sqrt(D)) V  within each sequence
 * q/out [total, H_q, D], k/v [total, H_kv, D] bf16 (innermost stride must be
 * 1, rows 16-byte aligned).  max_seqlen is the host-side longest length and
 * total_tokens = q.shape[0].  Allocates nothing; one kernel launch.
 * workspace: NULL / 0 bytes, or at least
 * wy_varlen_causal_prefill_workspace_bytes(batch, num_kv_heads, max_seqlen)
 * bytes of 4-byte aligned device memory holding two int32 counters that are
 * zero before the first call (each call leaves them zero).  With it a
 * persistent grid of one workgroup per CU draws the active query blocks,
 * heaviest first, from a shared ticket counter; without it there is one
 * workgroup per query block.  Results are identical.  Calls that may run
 * concurrently need distinct workspaces.
 * Replaces wy_lib::gqa_attention_varlen_causal
 *   (triton_kernels/gqa_attention_varlen_causal.py:214-278, kernel :101-210).
 */
int wy_varlen_causal_prefill(const void *q, const int64_t *q_strides,
                             const void *k, const int64_t *k_strides,
                             const void *v, const int64_t *v_strides, void *out,
                             const int64_t *out_strides,
                             const int32_t *cu_seqlens, int batch,
                             int num_q_heads, int num_kv_heads, int head_dim,
                             int max_seqlen, int64_t total_tokens, void *workspace,
                             int64_t workspace_bytes, void *stream);

/*
 * Workspace bytes wy_varlen_causal_prefill uses for its queue launch on the
 * current device: 8 (two int32 counters), or 0 when the grid of
 * ceil(max_seqlen / 32) * batch * num_kv_heads query blocks fits the device's
 * CUs in one round or 2 batch + ceil(max_seqlen / 32) + 2 exceeds 4096 (then the
 * one-workgroup-per-block launch is used).  No counterpart in the reference
 * (its launch takes no workspace).
 */
int64_t wy_varlen_causal_prefill_workspace_bytes(int batch, int num_kv_heads, int max_seqlen);

/*
 * Test hook, no counterpart in the reference: the order in which later
 * wy_varlen_causal_prefill / wy_prefill_attention_block launches (both the
 * one-workgroup-per-block and the queue launch) hand out their query blocks.
 * 0 (default) heaviest first, 1 lightest first, 2 alternately from both ends;
 * other values select 0.  Results do not depend on it (tests check this bit
 * for bit).  Process-wide; not for concurrent use with running launches.
 */
void wy_prefill_set_ticket_order(int order);

/*
 * Test hook, no counterpart in the reference: whether later
 * wy_varlen_causal_prefill / wy_prefill_attention_block launches whose grid of
 * query blocks fits the chip in one round and whose sequences are at most 128
 * tokens take the eight-wave short-sequence kernel (1, the default) or the
 * four-wave kernel (0).  The two agree within rounding, not bit for bit.
 * Process-wide; not for concurrent use with running launches.
 */
void wy_prefill_set_short_path(int enable);

/*
 * Prefill attention block: the reference's prefill attention sequence after
 * the q/k RMSNorm (engine/runner.py:336-384) in two launches, bit-identical
 * to it.  Replaces, in order:
 *   partial_rope(q), partial_rope(k)   (triton_kernels/partial_rope.py:145-198)
 *   gqa_attention_varlen_causal        (triton_kernels/gqa_attention_varlen_causal.py:214-278)
 *   attention_gate_pack                (triton_kernels/attention_gate_pack.py:77-126)
 *   paged_kv_fill_varlen               (triton_kernels/gqa_attention_decode_paged.py:492-561)
 * q [T, H_q, D], k / v [T, H_kv, D] (after q/k norm; unit inner stride, rows
 * 16-byte aligned), gate [T, H_q, D] view (unit inner stride, 16-byte aligned
 * rows), position_ids [T] (element stride pos_stride; int32, or int64 with
 * pos_is_int64 = 1), inv_freq [rotary_dim / 2] fp32, rotary_dim 64.
 * Launch 1 rotates K, writes K and V into the pages (block_table /
 * cu_seqlens as in wy_paged_kv_fill_varlen), the roped K into k_roped
 * ([T, H_kv, D] contiguous) and each token's sin / cos into rope_table
 * ([T][rotary_dim] fp32: sin of the rotary_dim/2 angles, then cos; 16-byte
 * aligned); both are caller-owned scratch.  Launch 2 is the varlen causal
 * attention with q's RoPE (from that table) applied at load and out [T, H_q * D]
 * (contiguous) = bf16(bf16(attention) * sigmoid(gate)).  workspace as in
 * wy_varlen_causal_prefill.  Allocates nothing.
 */
int wy_prefill_attention_block(const void *q, const int64_t *q_strides, const void *k,
                               const int64_t *k_strides, const void *v,
                               const int64_t *v_strides, const void *gate,
                               const int64_t *gate_strides, const void *position_ids,
                               int64_t pos_stride, int pos_is_int64, const float *inv_freq,
                               int rotary_dim, void *k_cache, void *v_cache,
                               const int64_t *kc_strides, const int64_t *vc_strides,
                               const int32_t *block_table, int64_t bt_stride0,
                               const int32_t *cu_seqlens, int batch, int num_q_heads,
                               int num_kv_heads, int head_dim, int max_seqlen,
                               int64_t total_tokens, void *k_roped, float *rope_table,
                               void *out, void *workspace, int64_t workspace_bytes,
                               void *stream);

/*
 * Launch 1 of wy_prefill_attention_block on its own: the varlen K/V page fill
 * with K rotated (partial RoPE on dims [0, rotary_dim), rotary_dim % 16 == 0, at most 128)
 * before it is written, to the pages and to k_roped ([T, H_kv, D], strides
 * kr_strides); rope_table (optional, NULL to skip) receives each token's
 * sin / cos as in wy_prefill_attention_block.  Equals partial_rope(k) followed by paged_kv_fill_varlen
 * (triton_kernels/partial_rope.py:145-198, gqa_attention_decode_paged.py:492-561).
 * Unit inner strides and 16-byte aligned rows everywhere (else WY_E_LAYOUT).
 */
int wy_prefill_kv_rope_fill(void *k_cache, void *v_cache, const int64_t *kc_strides,
                            const int64_t *vc_strides, const void *k, const int64_t *k_strides,
                            const void *v, const int64_t *v_strides, void *k_roped,
                            const int64_t *kr_strides, float *rope_table,
                            const int32_t *block_table,
                            int64_t bt_stride0, const int32_t *cu_seqlens,
                            const void *position_ids, int64_t pos_stride, int pos_is_int64,
                            const float *inv_freq, int rotary_dim, int batch, int num_kv_heads,
                            int head_dim, int max_seqlen, void *stream);

/*
 * Partial rotate-half RoPE on dims [0, rotary_dim) of x [B, H, T, D] bf16;
 * dims [rotary_dim, D) are copied bit-exactly.  angle = float(pos) * inv_freq[j]
 * in fp32.  position_ids [B, T] is int32 (pos_is_int64 = 0) or int64 (= 1).
 * x_strides / out_strides / pos_strides are element strides.
 * Replaces wy_lib::partial_rope
 *   (triton_kernels/partial_rope.py:145-198, kernel :34-132).
 */
int wy_partial_rope(const void *x, const int64_t *x_strides, void *out,
                    const int64_t *out_strides, const void *position_ids,
                    const int64_t *pos_strides, int pos_is_int64,
                    const float *inv_freq, int batch, int num_heads,
                    int num_tokens, int head_dim, int rotary_dim, void *stream);

/*
 * Sigmoid output gate + head packing:
 *   out[t, h*D + d] = bf16(float(x[0,h,t,d]) * sigmoid(float(gate[0,h,t,d])))
 * x, gate [1, H, T, D] bf16 with any strides; out [T, H*D] contiguous.
 * Replaces wy_lib::attention_gate_pack
 *   (triton_kernels/attention_gate_pack.py:77-126, kernel :20-63).
 */
int wy_attention_gate_pack(const void *x, const int64_t *x_strides,
                           const void *gate, const int64_t *gate_strides,
                           void *out, int num_heads, int num_tokens,
                           int head_dim, void *stream);

/*
 * Per-row RMSNorm with a (1 + w) weight:
 *   out[b, m, :] = bf16(x * rsqrt(mean(x^2) + eps) * (1 + weight))  (fp32 math)
 * x [batch, rows, d_model] bf16 with strides x_strides (innermost 1, rows
 * 16-byte aligned); weight [d_model] bf16; out [batch, rows, d_model] with
 * out_strides.  d_model a multiple of 256.
 * Replaces wy_lib::qwen_rmsnorm
 *   (triton_kernels/qwen_rmsnorm.py:92-147, kernel :28-90).
 */
int wy_qwen_rmsnorm(const void *x, const int64_t *x_strides, const void *weight,
                    void *out, const int64_t *out_strides, int batch, int rows,
                    int d_model, float eps, void *stream);

/*
 * Decode attention block in one launch: from the fused projection's raw
 * q / gate / k / v slices to the gated, head-packed attention output.
 *   q = rope(rmsnorm(q_raw, q_norm_weight)), k = rope(rmsnorm(k_raw, k_norm_weight))
 *   at position pos[b] on dims [0, rotary_dim), v = v_raw; append k, v at pos;
 *   split-K attention + merge; out = bf16(bf16(ctx) * sigmoid(gate)).
 * q_raw, gate [B, H_q, D] and k_raw, v_raw [B, H_kv, D] bf16 with any row
 * strides (innermost 1), e.g. views of the [B, 5120] projection output;
 * weights [D] bf16; inv_freq [rotary_dim/2] fp32; rotary_dim <= 128, a multiple of
 * 16.  Caches, table, scratch and counters as wy_paged_decode_step; out
 * [B, H_q, D] (the packed [B, H_q*D] row when contiguous).  Bit-identical to
 * wy_qwen_rmsnorm + wy_partial_rope + wy_paged_decode_step in sequence.
 * Replaces the sequence qwen_rmsnorm(q), qwen_rmsnorm(k), partial_rope(q),
 * partial_rope(k), call_paged_gqa_attention_decode_triton, attention_gate_pack
 * of engine/runner.py:476-517.
 */
int wy_paged_decode_block(const void *q_raw, const int64_t *q_strides, const void *gate,
                          const int64_t *gate_strides, const void *k_raw,
                          const int64_t *k_strides, const void *v_raw,
                          const int64_t *v_strides, const void *q_norm_weight,
                          const void *k_norm_weight, float eps, const float *inv_freq,
                          int rotary_dim, void *k_cache, void *v_cache,
                          const int64_t *kc_strides, const int64_t *vc_strides,
                          const int32_t *block_table, int64_t bt_stride0,
                          const int64_t *pos, float *m_partial, float *l_partial,
                          float *acc_partial, const int64_t *ml_strides,
                          const int64_t *acc_strides, int32_t *counters, void *out,
                          const int64_t *out_strides, int batch, int num_q_heads,
                          int num_kv_heads, int head_dim, int max_pages,
                          int min_pages_per_split, void *stream);

/*
 * Projection GEMM:  y[m, n] = bf16(sum_k x[m, k] * w[n, k])  (fp32 accumulation)
 * x [M, K], w [N, K], y [M, N] bf16, row strides x_strides[0] / w_strides[0] /
 * y_strides[0] (elements; x and w rows 16-byte aligned), inner strides 1;
 * K a multiple of 128.  M <= 64 runs a weight-streaming kernel, larger M a
 * 128 x 128-tile MFMA kernel.  Allocates nothing; one kernel launch.
 * workspace: NULL / 0 bytes, or at least wy_gemm_2d_workspace_bytes(M, N, K)
 * bytes of 4-byte aligned device memory whose first 16 KiB are zero before
 * the first call (each call leaves them zero).  With it, weight-streaming
 * shapes with few column blocks split K across workgroups (fp32 partials
 * summed in split order by the last workgroup of each column block);
 * without it each column block is one workgroup.  Calls that may run
 * concurrently need distinct workspaces.
 * Replaces wy_lib::gemm_2d (triton_kernels/gemm_2d.py:197-230, kernel :157-195).
 */
int wy_gemm_2d(const void *x, const int64_t *x_strides, const void *w,
               const int64_t *w_strides, void *y, const int64_t *y_strides, int M, int N,
               int K, void *workspace, int64_t workspace_bytes, void *stream);

/*
 * Workspace bytes wy_gemm_2d uses to split K for this shape: 16 KiB of
 * counters + split * M * N * 4 bytes of partials, or 0 when it does not
 * split.  No counterpart in the reference (its launch takes no workspace).
 */
int64_t wy_gemm_2d_workspace_bytes(int M, int N, int K);

/*
 * Gated DeltaNet delta-rule decode: one token per sequence, the fp32 state
 * updated in place.  For each (b, h):  S = exp(g) S;  delta = beta (v - k^T S);
 * S += k delta^T;  out = bf16(q^T S).
 * q, k [B, H, key_dim], v, out [B, H, value_dim] bf16 (element strides, any);
 * beta, g [B, H] fp32; state [B, H, key_dim, value_dim] fp32 (unit inner
 * stride, 16-byte aligned rows).  key_dim 128, value_dim a multiple of 128
 * (else WY_E_UNSUPPORTED).  Allocates nothing; one launch.
 * Replaces wy_lib::gdn_recurrent_decode
 *   (triton_kernels/gdn_recurrent_prefill.py:1185-1260, kernel :151-246).
 */
int wy_gdn_recurrent_decode(const void *q, const int64_t *q_strides, const void *k,
                            const int64_t *k_strides, const void *v, const int64_t *v_strides,
                            const float *beta, const int64_t *beta_strides, const float *g,
                            const int64_t *g_strides, void *out, const int64_t *out_strides,
                            float *state, const int64_t *state_strides, int batch,
                            int num_heads, int key_dim, int value_dim, void *stream);

/*
 * Gated DeltaNet chunk-64 (WY) prefill of one prompt, stage 1 of 3: per chunk
 * of 64 tokens and head, G = cumsum(g) (g_cumsum [N, H, 64]), and the
 * solutions of (I + L) X = B with L[t, i] = beta_t exp(G_t - G_i) <k_t, k_i>
 * (i < t): u_base = X for B = beta v ([N, H, 64, value_dim]), w = X for
 * B = beta exp(G) k ([N, H, 64, key_dim]); all fp32, contiguous, N =
 * ceil(T/64).  Rows past T: w and u_base are zero; g_cumsum repeats the last
 * valid cumulative value (the reference's unmasked store writes the same).  k, v [T, H, 128] bf16 (unit inner stride,
 * 16-byte aligned rows), beta, g [T, H] fp32.  key_dim = value_dim = 128.
 * Replaces wy_lib::gdn_chunk_prepare_wy
 *   (triton_kernels/gdn_recurrent_prefill.py:703-826, kernel :249-402).
 */
int wy_gdn_chunk_prepare_wy(const void *k, const int64_t *k_strides, const void *v,
                            const int64_t *v_strides, const float *beta,
                            const int64_t *beta_strides, const float *g,
                            const int64_t *g_strides, float *w, float *u_base, float *g_cumsum,
                            int token_num, int num_heads, int key_dim, int value_dim,
                            void *stream);

/*
 * Stage 2: the chunk recurrence.  chunk_state[c] = the state entering chunk
 * c ([N, H, key_dim, value_dim]), delta = u_base - w S ([N, H, 64, value_dim]),
 * S = exp(G_last) S + k^T (delta exp(G_last - G_t)) with tokens past T
 * masked; final_state [H, key_dim, value_dim].  All fp32 contiguous.
 * Replaces wy_lib::gdn_chunk_state
 *   (triton_kernels/gdn_recurrent_prefill.py:829-936, kernel :405-562).
 */
int wy_gdn_chunk_state(const void *k, const int64_t *k_strides, const float *w,
                       const float *u_base, const float *g_cumsum, float *delta,
                       float *chunk_state, float *final_state, int token_num, int num_heads,
                       int key_dim, int value_dim, void *stream);

/*
 * Stage 3: out_t = exp(G_t) q_t S_c + sum_{i <= t in the chunk}
 * exp(G_t - G_i) <q_t, k_i> delta_i, stored bf16 [T, H, value_dim] with
 * out_strides (unit inner stride).  q, k as stage 1.
 * Replaces wy_lib::gdn_chunk_output
 *   (triton_kernels/gdn_recurrent_prefill.py:939-1023, kernel :565-690).
 */
int wy_gdn_chunk_output(const void *q, const int64_t *q_strides, const void *k,
                        const int64_t *k_strides, const float *delta, const float *g_cumsum,
                        const float *chunk_state, void *out, const int64_t *out_strides,
                        int token_num, int num_heads, int key_dim, int value_dim,
                        void *stream);

/*
 * Gated DeltaNet sequential prefill over a packed varlen batch: sequence b
 * owns tokens [cu_seqlens[b], cu_seqlens[b+1]) of q, k [T, H, key_dim],
 * v, out [T, H, value_dim] (bf16), beta, g [T, H] fp32, and starts from a
 * zero state; its final state goes to state[b] ([B, H, key_dim, value_dim]
 * fp32, unit inner stride).  cu_seqlens [B+1] int32 on the device.  Same
 * step as wy_gdn_recurrent_decode.  Allocates nothing; one launch.
 * Replaces wy_lib::gdn_recurrent_prefill_sequential
 *   (triton_kernels/gdn_recurrent_prefill.py:1050-1146, kernel :52-143).
 */
int wy_gdn_recurrent_prefill_sequential(const void *q, const int64_t *q_strides, const void *k,
                                        const int64_t *k_strides, const void *v,
                                        const int64_t *v_strides, const float *beta,
                                        const int64_t *beta_strides, const float *g,
                                        const int64_t *g_strides, void *out,
                                        const int64_t *out_strides, float *state,
                                        const int64_t *state_strides,
                                        const int32_t *cu_seqlens, int batch, int num_heads,
                                        int key_dim, int value_dim, void *stream);

/*
 * Depthwise causal conv (4 taps) decode step + SiLU.  x [B, C] bf16 (element
 * strides); state [B, 4, C] bf16 (unit channel stride) holds the last four
 * conv inputs and is shifted in place (x enters at tap 3); weight [4, C] bf16
 * (unit channel stride).  out[b, c] = bf16(silu(sum_r w[r, c] * state'[b, r, c]))
 * with fp32 accumulation in tap order.  Allocates nothing; one launch.
 * Replaces wy_lib::depthwise_causal_conv4_decode
 *   (triton_kernels/depthwise_causal_conv4_decode.py:152-205, kernel :86-150).
 */
int wy_depthwise_causal_conv4_decode(const void *x, const int64_t *x_strides, void *state,
                                     const int64_t *state_strides, const void *weight,
                                     const int64_t *w_strides, void *out,
                                     const int64_t *out_strides, int batch, int channels,
                                     void *stream);

/*
 * GDN q/k L2 norm and gates.  q, k [T, H, D] bf16 (element strides), a, b
 * [T, H] bf16, a_log [H] fp32, dt_bias [H] bf16.  Writes q_norm, k_norm
 * ([T, H, D] contiguous bf16): q * rsqrt(sum q^2 + 1e-6) * D^-1/2 and
 * k * rsqrt(sum k^2 + 1e-6); beta, g ([T, H] contiguous fp32):
 * sigmoid(b) and -exp(a_log) * softplus(a + dt_bias).  D = 128.
 * Replaces wy_lib::gdn_qk_norm_gates
 *   (triton_kernels/gdn_qk_norm_gates.py:127-201, kernel :19-115).
 */
int wy_gdn_qk_norm_gates(const void *q, const int64_t *q_strides, const void *k,
                         const int64_t *k_strides, const void *a, const int64_t *a_strides,
                         const void *b, const int64_t *b_strides, const float *a_log,
                         const void *dt_bias, void *q_norm, void *k_norm, float *beta, float *g,
                         int tokens, int num_heads, int head_dim, void *stream);

/*
 * GDN gated RMSNorm.  x, z [T, H, D] bf16 (element strides), weight [D] fp32;
 * out [T, H, D] contiguous bf16 = x * rsqrt(mean(x^2) + 1e-6) * w * z * sigmoid(z).
 * D = 128.
 * Replaces wy_lib::gdn_gated_rmsnorm
 *   (triton_kernels/gdn_gated_rmsnorm.py:88-137, kernel :21-76).
 */
int wy_gdn_gated_rmsnorm(const void *x, const int64_t *x_strides, const void *z,
                         const int64_t *z_strides, const float *weight, void *out, int tokens,
                         int num_heads, int head_dim, void *stream);

/*
 * GDN decode mixer in one launch, from the fused projection row to the
 * out_proj input: conv4 decode + SiLU of the q/k/v channels (conv_state
 * shifted in place), q/k L2 norm and gates, one delta-rule step (state
 * advanced in place), gated RMSNorm.  Equals, bit for bit, the sequence
 * wy_depthwise_causal_conv4_decode -> wy_gdn_qk_norm_gates ->
 * wy_gdn_recurrent_decode -> wy_gdn_gated_rmsnorm.
 * fused [B, 3HD + HD + 2H] bf16 (row stride fused_stride0): q|k|v conv
 * inputs, z, a, b as the reference's in_proj_fused rows; conv_state
 * [B, 4, 3HD] bf16; conv_weight [4, 3HD] bf16; a_log [H] fp32; dt_bias [H]
 * bf16; norm_weight [D] fp32; state [B, H, D, D] fp32 (unit inner stride,
 * 16-byte rows); out [B, H*D] bf16 (row stride out_stride0).  D = 128.
 * Replaces the runner's GDN decode sequence between the fused projection and
 * out_proj (engine/runner.py:431-441): depthwise_causal_conv4_decode,
 * gdn_qk_norm_gates, gdn_recurrent_decode, gdn_gated_rmsnorm.
 */
int wy_gdn_decode_block(const void *fused, int64_t fused_stride0, void *conv_state,
                        const int64_t *conv_state_strides, const void *conv_weight,
                        int64_t conv_weight_stride0, const float *a_log, const void *dt_bias,
                        const float *norm_weight, float *state, const int64_t *state_strides,
                        void *out, int64_t out_stride0, int batch, int num_heads, int head_dim,
                        void *stream);

/*
 * Depthwise causal conv (4 taps) + SiLU over a prompt, optionally packed:
 * out[t, c] = bf16(silu(sum_r w[c, r] * x[t - 3 + r, c])), taps before
 * seq_start[t] (or before 0 when seq_start is NULL) read as zero.  x, out
 * [T, C] bf16 (element strides); weight element (c, r) at
 * c * w_stride_c + r * w_stride_k ([C, 4] or [C, 1, 4]); seq_start [T] int32.
 * Same arithmetic as wy_depthwise_causal_conv4_decode.  One launch.
 * Replaces wy_lib::depthwise_causal_conv4_prefill
 *   (triton_kernels/depthwise_causal_conv4_prefill.py:104-176, kernel :23-92).
 */
int wy_depthwise_causal_conv4_prefill(const void *x, const int64_t *x_strides,
                                      const void *weight, int64_t w_stride_c,
                                      int64_t w_stride_k, void *out, const int64_t *out_strides,
                                      const int32_t *seq_start, int tokens, int channels,
                                      void *stream);

/*
 * Decode conv states after a packed prefill: state[b, r, :] = x[end_b - 4 + r, :]
 * (end_b = cu_seqlens[b+1]), zero where that row lies before cu_seqlens[b].
 * state [B, 4, C] bf16 (unit channel stride), x [T, C] bf16 (unit channel
 * stride).  Replaces wy_lib::conv_state_from_packed_prefill
 *   (triton_kernels/depthwise_causal_conv4_decode.py:332-375, kernel :253-330).
 */
int wy_conv_state_from_packed_prefill(void *state, const int64_t *state_strides, const void *x,
                                      const int64_t *x_strides, const int32_t *cu_seqlens,
                                      int batch, int channels, void *stream);

/*
 * Token embedding gather: out[t, :] = weight[input_ids[t], :] (bf16 rows of
 * d_model, d_model % 8 == 0, 16-byte aligned rows); input_ids [T] int32 or
 * int64 (ids_is_int64); weight has `vocab` rows, and an id outside [0, vocab)
 * writes a zero row (never a read past the table).  Replaces
 * wy_lib::embedding_gather (triton_kernels/embedding_gather.py:62-104, kernel :20-50).
 */
int wy_embedding_gather(const void *input_ids, int ids_is_int64, const void *weight,
                        int64_t weight_row_stride, int64_t vocab, void *out,
                        int64_t out_row_stride, int tokens, int d_model, void *stream);

/*
 * out = bf16(x + residual) over n contiguous bf16 elements (16-byte aligned).
 * Replaces wy_lib::residual_add (triton_kernels/residual_add.py:23-52, kernel :8-20).
 */
int wy_residual_add(const void *x, const void *residual, void *out, int64_t n, void *stream);

/*
 * Residual add fused with the following RMSNorm: sum = bf16(h + x) and
 * out = bf16(sum * rsqrt(mean(sum^2) + eps) * (1 + weight)), fp32 math, over
 * [rows, d_model] contiguous bf16 rows (16-byte aligned, d_model a multiple
 * of 256 up to 1024).  Equals wy_residual_add -> wy_qwen_rmsnorm bit for bit.
 * sum and out must not alias h, x or each other.  No single counterpart in
 * the reference: it fuses the residual_add -> qwen_rmsnorm pairs of its
 * decoder layer loop (engine/runner.py:555-558, :566-571; prefill :650-663)
 * into one launch.
 */
int wy_add_rmsnorm(const void *h, const void *x, const void *weight, void *sum, void *out,
                   int rows, int d_model, float eps, void *stream);

/*
 * SwiGLU: out[m, n] = bf16(up * gate * sigmoid(gate)), fp32 math; gate, up
 * [rows, cols] bf16 (element strides), out [rows, cols] contiguous.
 * Replaces wy_lib::swiglu (triton_kernels/swiglu.py:72-111, kernel :22-60).
 */
int wy_swiglu(const void *gate, const int64_t *gate_strides, const void *up,
              const int64_t *up_strides, void *out, int rows, int cols, void *stream);

/*
 * LM head fused with the vocabulary argmax: token_ids[m] = argmax_v
 * sum_k hidden[m, k] * weight[v, k] (fp32 sums, the first index on ties;
 * NaN ranks above every number, first NaN wins, as torch.argmax; the result
 * is always in [0, vocab)), logits never written.  hidden [rows, hidden_size] bf16 (rows <= 64),
 * weight [vocab, hidden_size] bf16, 16-byte aligned rows; hidden_size a
 * multiple of 256; token_ids [rows] int64.  workspace: at least
 * wy_lm_head_argmax_workspace_bytes(rows, hidden_size, vocab) bytes,
 * 8-byte aligned, no initial contents.  Two launches.
 * Replaces wy_lib::lm_head_argmax (triton_kernels/vocab_argmax.py:137-224,
 * kernels :29-135).
 */
int wy_lm_head_argmax(const void *hidden, int64_t hidden_row_stride, const void *weight,
                      int64_t weight_row_stride, int64_t *token_ids, int rows, int hidden_size,
                      int vocab, void *workspace, int64_t workspace_bytes, void *stream);

/* Workspace bytes wy_lm_head_argmax needs (per-workgroup partial keys).  No
 * counterpart in the reference (its op allocates the partials itself). */
int64_t wy_lm_head_argmax_workspace_bytes(int rows, int hidden_size, int vocab);

/*
 * wy_gemm_2d with the RMSNorm in the A-operand load: y = bf16(qwen_rmsnorm(t)
 * @ w^T) with t = bf16(x + residual) (residual may be NULL: t = x) and
 * qwen_rmsnorm(t) = bf16(t * rsqrt(mean(t^2) + eps) * (1 + norm_weight)),
 * the same roundings and reduction order as wy_qwen_rmsnorm; when x_out is
 * not NULL it receives t (the residual stream).  Equals wy_residual_add ->
 * wy_qwen_rmsnorm -> wy_gemm_2d bit for bit.  M <= 64 (else
 * WY_E_UNSUPPORTED), K % 256 == 0, rows 16-byte aligned; x_out must not
 * alias x or residual.  workspace as in wy_gemm_2d.  One launch.
 * No counterpart in the reference: it fuses residual_add + qwen_rmsnorm +
 * gemm_2d of the runner's decode step (engine/runner.py:538-562).
 */
int wy_gemm_2d_rmsnorm(const void *x, int64_t x_stride0, const void *residual,
                       int64_t residual_stride0, const void *norm_weight, float eps, void *x_out,
                       int64_t x_out_stride0, const void *w, int64_t w_stride0, void *y,
                       int64_t y_stride0, int M, int N, int K, void *workspace,
                       int64_t workspace_bytes, void *stream);

/*
 * wy_gemm_2d with SwiGLU in the A-operand load: y = bf16(swiglu(gate, up) @ w^T)
 * where gate = gate_up[:, 0:K], up = gate_up[:, up_offset:up_offset+K] and
 * swiglu = bf16(up * gate * sigmoid(gate)) as wy_swiglu.  Equals wy_swiglu ->
 * wy_gemm_2d bit for bit.  M <= 64.  No counterpart in the reference: it fuses
 * swiglu + the down projection (engine/runner.py:562-565).
 */
int wy_gemm_2d_swiglu(const void *gate_up, int64_t gate_up_stride0, int64_t up_offset,
                      const void *w, int64_t w_stride0, void *y, int64_t y_stride0, int M, int N,
                      int K, void *workspace, int64_t workspace_bytes, void *stream);

/*
 * The gate/up projection with SwiGLU in the epilogue: w [2N, K] holds the gate
 * rows [0, N) and the up rows [N, 2N); y [M, N] = bf16(up * gate *
 * sigmoid(gate)) with gate = bf16(x @ w[0:N]^T), up = bf16(x @ w[N:2N]^T).
 * Equals wy_gemm_2d (x, w) -> wy_swiglu bit for bit, except for M <= 64 with
 * 2N < 4096 (another workgroup plan: fp32 summation order differs).
 * M <= 64 (decode) or N % 128 == 0 (else WY_E_UNSUPPORTED), K % 128 == 0,
 * rows 16-byte aligned;
 * workspace as in wy_gemm_2d, sized by
 * wy_gemm_2d_gate_up_swiglu_workspace_bytes.  No counterpart in the
 * reference: it fuses the gate_up gemm_2d and swiglu of its MLP
 * (engine/runner.py:560-565) into one launch.
 */
int wy_gemm_2d_gate_up_swiglu(const void *x, int64_t x_stride0, const void *w,
                              int64_t w_stride0, void *y, int64_t y_stride0, int M, int N, int K,
                              void *workspace, int64_t workspace_bytes, void *stream);

/* Workspace bytes wy_gemm_2d_gate_up_swiglu needs for split K (0: none). */
int64_t wy_gemm_2d_gate_up_swiglu_workspace_bytes(int M, int N, int K);

#ifdef __cplusplus
}
#endif

#endif /* WY_ATTN_H */
