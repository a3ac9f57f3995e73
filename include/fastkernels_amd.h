/*
 * fastkernels_amd.h — C ABI of the MI355X (gfx950) decode-step operator library.
 *
 * One shared library, libfk_amd.so, exports one entry point per operator of the
 * serving-engine decode step.  Every entry point:
 *   - takes raw device pointers, element counts, row strides (in elements) and a
 *     hipStream_t passed as void* (NULL = the null stream);
 *   - enqueues its kernels on that stream and returns without synchronising;
 *   - allocates nothing (the paged-decode split-context workspace is caller-owned);
 *   - returns FK_OK (0), a negative FK_ERR_* code for a rejected argument, or a
 *     positive hipError_t from the launch.  fk_last_error() returns a message for
 *     the last failing call on the calling thread.
 * No torch types appear here: the Python layer (fastkernels_amd/_native.py)
 * binds these symbols with ctypes.
 *
 * Reference interfaces replaced (paths relative to the Snowflake-AI-Research/
 * fastkernels checkout):
 *   fk_rmsnorm / fk_fused_add_rmsnorm
 *       fastkernels/tasks/baseline/L1/rms_norm.py:44-69 (ops fastkernels_norm::rmsnorm,
 *       fastkernels_norm::fused_add_rmsnorm) and the vLLM kernels they bind,
 *       rms_norm.cu:1456 (rms_norm) and rms_norm.cu:1546 (fused_add_rms_norm).
 *   fk_rotary_embedding
 *       fastkernels/tasks/baseline/L1/rotary_emb.py:24-39 (op fastkernels_rope::rotary_embedding),
 *       host function rotary_emb.cu:427-533.
 *   fk_store_kvcache
 *       fastkernels/tasks/baseline/L1/store_kvcache.py:16-35,71-82 (Triton _store_kvcache_kernel,
 *       StoreKVCache.forward, NHD layout).
 *   fk_paged_decode_plan / fk_paged_decode (+ _partials / _reduce phases)
 *       fastkernels/tasks/baseline/L1/flash_attn_decode.py:113-181 (FlashAttnDecode.forward ->
 *       vllm.vllm_flash_attn.flash_attn_varlen_func with block_table, seqused_k, num_splits);
 *       split-context merge semantics of triton_unified_attention.py:697-784 (reduce_segments);
 *       fp8 per-tensor KV dequant semantics of triton_unified_attention.py:51-67 (_cast_kv_tile).
 *   fk_silu_and_mul
 *       fastkernels/tasks/baseline/L1/silu_and_mul.py:24-30 (_C.silu_and_mul(out, x)),
 *       kernel silu_and_mul.cu:951-956.
 *   fk_merge_attn_states
 *       fastkernels/tasks/baseline/L1/merge_attn_states.py:30-122 (merge_attn_states,
 *       MergeAttnStates.forward).
 *   fk_store_paged_decode
 *       fastkernels/tasks/baseline/L2/attention_impl.py:313-363 (forward_impl: store,
 *       then the decode branch of _forward_pure :436-450).
 *   fk_store_kvcache_convert
 *       fastkernels/tasks/baseline/L1/store_kvcache.py:16-35,71-82 (StoreKVCache.forward
 *       when key and cache dtypes differ).
 *   fk_store_kvcache_hnd
 *       fastkernels/tasks/baseline/L1/store_kvcache.py:36-68,85-99 (Triton
 *       _store_kvcache_hnd_kernel, StoreKVCacheHND.forward, HND layout).
 *   fk_paged_prefill, fk_varlen_prefill
 *       fastkernels/tasks/baseline/L1/flash_attn_prefill.py:18-74 (FlashAttnPrefill.forward,
 *       with and without block_table).
 *   fk_qk_norm_rope_store
 *       fastkernels/tasks/baseline/L2/attention.py:120-140 (q_norm/k_norm, rotary_emb)
 *       followed by attention_impl.py:323-325 (store_kvcache).
 */
#ifndef FASTKERNELS_AMD_H_
#define FASTKERNELS_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (negative = argument rejected before any launch). */
#define FK_OK 0
#define FK_ERR_INVALID_ARG (-1)
#define FK_ERR_UNSUPPORTED (-2)
#define FK_ERR_WORKSPACE (-3)

/* Element type tags. */
#define FK_DTYPE_F32 0
#define FK_DTYPE_F16 1
#define FK_DTYPE_BF16 2
#define FK_DTYPE_FP8_E4M3FN 3 /* OCP float8 e4m3fn (torch.float8_e4m3fn) */

/* Library version as 10000*major + 100*minor + patch.  The major version changes
 * whenever an existing entry point's signature changes; a caller built against this
 * header checks fk_version() / 10000 == FK_VERSION_MAJOR before binding. */
#define FK_VERSION_MAJOR 2
#define FK_VERSION_MINOR 1 /* 2.1: fk_prefill_split_plan, fk_paged_prefill_ws, fk_varlen_prefill_ws */
int fk_version(void);

/* Message describing the last failing call on this thread ("" if none). */
const char* fk_last_error(void);

/* RMSNorm without residual: out[r,:] = cast(x[r,:] * rsqrt(mean(x[r,:]^2) + eps)) * weight.
 * x rows are `x_row_stride` elements apart, out rows `out_row_stride`; the
 * hidden dimension is contiguous.  dtype is F32, F16 or BF16 for x/out/weight.
 * Replaces fastkernels_norm::rmsnorm (rms_norm.py:51) / vLLM rms_norm (rms_norm.cu:1456). */
int fk_rmsnorm(void* out, int64_t out_row_stride, const void* x, int64_t x_row_stride,
               const void* weight, int64_t rows, int64_t hidden, float eps, int dtype,
               void* stream);

/* Fused residual add + RMSNorm, in place on both tensors:
 *   residual[r,:] <- cast(x[r,:] + residual[r,:])            (sum formed in fp32)
 *   x[r,:]        <- cast(cast(s * rsqrt(mean(s^2) + eps)) * weight),  s = fp32 sum
 * Replaces fastkernels_norm::fused_add_rmsnorm (rms_norm.py:57-65) and vLLM
 * fused_add_rms_norm (rms_norm.cu:1546-1598); numerics follow forward_native
 * (rms_norm.py:97-118). */
int fk_fused_add_rmsnorm(void* x, int64_t x_row_stride, void* residual,
                         int64_t residual_row_stride, const void* weight, int64_t rows,
                         int64_t hidden, float eps, int dtype, void* stream);

/* Rotary embedding, in place on query and (optional, may be NULL) key.
 * positions: int64 [tokens].  query rows `q_row_stride` elements apart, each row
 * num_heads*head_size contiguous; same for key with num_kv_heads.
 * cos_sin: [max_position, rot_dim] rows (first rot_dim/2 = cos, rest = sin) of
 * dtype `cache_dtype` (F32 or the query dtype).  cos/sin are rounded to the query
 * dtype before use, as the reference casts the cache (rotary_emb.py:171-173).
 * is_neox != 0: pairs (i, i + rot_dim/2); else pairs (2i, 2i+1).
 * Positions outside [0, max_position) leave that token unchanged.
 * Replaces fastkernels_rope::rotary_embedding (rotary_emb.py:26-37). */
int fk_rotary_embedding(const int64_t* positions, void* query, int64_t q_row_stride,
                        void* key, int64_t k_row_stride, const void* cos_sin,
                        int cache_dtype, int64_t max_position, int64_t tokens,
                        int num_heads, int num_kv_heads, int head_size, int rot_dim,
                        int is_neox, int dtype, void* stream);

/* store_kvcache (NHD paged layout), a bit-exact scatter:
 *   for i < tokens with s = slot_mapping[i] >= 0:
 *     k_cache[s*row_elems : (s+1)*row_elems] = key[i*key_row_stride : +row_elems]
 *     v_cache[...]                           = value[i*value_row_stride : +row_elems]
 * row_elems = num_kv_heads*head_size, elem_bytes = bytes per element (1, 2 or 4).
 * slot_mapping is int64 when slot_is_i64 != 0, else int32.  Slots >= num_slots
 * (= num_blocks*block_size) are skipped like negative ones, so no write leaves
 * the cache.  Replaces StoreKVCache.forward (store_kvcache.py:71-82). */
int fk_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                     int64_t value_row_stride, void* k_cache, void* v_cache,
                     const void* slot_mapping, int slot_is_i64, int64_t tokens,
                     int64_t row_elems, int elem_bytes, int64_t num_slots, void* stream);

/* store_kvcache into the HND paged layout [num_blocks, num_kv_heads, page_size,
 * head_size] (a bit-exact scatter): for i < tokens with s = slot_mapping[i] in
 * [0, num_slots), head h's row of key/value goes to
 *   cache[((s / page_size) * num_kv_heads + h) * page_size + s % page_size][0 : head_size].
 * key/value rows `*_row_stride` elements apart, heads head_size apart within a row.
 * Slots outside [0, num_slots) are skipped.  elem_bytes 1, 2 or 4.
 * Replaces StoreKVCacheHND.forward (store_kvcache.py:85-99, kernel :36-68). */
int fk_store_kvcache_hnd(const void* key, int64_t key_row_stride, const void* value,
                         int64_t value_row_stride, void* k_cache, void* v_cache,
                         const void* slot_mapping, int slot_is_i64, int64_t tokens,
                         int num_kv_heads, int head_size, int page_size, int elem_bytes,
                         int64_t num_slots, void* stream);

/* Chooses the schedule of a paged-decode launch (host-only; may query the
 * device's CU count once).  Outputs:
 *   part_tokens: 0 = length-balanced schedule (the default, num_splits == 0):
 *                the tiles of all sequences are cut into max_parts equal
 *                ranges, one work-group each;
 *                > 0 = fixed partitions of part_tokens tokens per sequence
 *                (num_splits > 0 asks for that many over max_seq_len, as
 *                flash_attn_varlen_func's num_splits).
 *   max_parts:   work-groups per kv-head group (balanced) or partitions per
 *                sequence (fixed).
 *   workspace_bytes: device workspace fk_paged_decode needs for this plan. */
int fk_paged_decode_plan(int64_t batch, int num_heads, int num_kv_heads, int head_size,
                         int64_t max_seq_len, int num_splits, int64_t* part_tokens,
                         int64_t* max_parts, int64_t* workspace_bytes);

/* Paged decode attention (one query token per sequence, at position ctx_lens[b] - 1):
 *   out[b,h,:] = softmax(scale * q[b,h,:] . K_b^T) V_b  over tokens [lo_b, ctx_lens[b])
 * of sequence b, gathered through block_tables[b, :]; kv head = h / (Hq/Hk).
 * window_left: -1 = every token (lo_b = 0); >= 0 = sliding window (flash-attn
 *    window_size = (window_left, 0)): lo_b = max(0, ctx_lens[b] - 1 - window_left).
 * sinks: NULL, or device fp32 [num_heads] attention-sink logits (flash-attn s_aux),
 *    in the units of scale * q . k: they join each row's softmax denominator only,
 *    out = sum_t e^(s_t - m) V_t / (sum_t e^(s_t - m) + e^(sink - m)); an empty row
 *    stays 0.
 * q: [batch, num_heads, head_size] rows `q_row_stride` elements apart (head_size
 *    contiguous, heads head_size apart); dtype BF16.
 * k_cache, v_cache: [num_blocks, block_size, num_kv_heads, head_size] of kv_dtype
 *    (BF16, or FP8_E4M3FN dequantised as float(x) * k_scale[kv_head] /
 *    v_scale[kv_head]; scale pointers are device fp32 [num_kv_heads] or NULL = 1).
 * block_tables: int32 [batch, bt_row_stride]; entries outside [0, num_blocks),
 *    and pages past the row (index >= bt_row_stride), are masked (never read).
 *    ctx_lens: int32 [batch]; 0 gives a zero output row.
 * out: [batch, num_heads, head_size] BF16 rows `out_row_stride` elements apart.
 * part_tokens / max_parts: from fk_paged_decode_plan.  With fixed partitions,
 *    partition p covers tokens [p * part_tokens, (p + 1) * part_tokens) and the
 *    last one runs on to the context end, so every key is attended whatever the
 *    plan's max_seq_len (a context longer than it makes the last partition
 *    longer); the balanced schedule reads the lengths on the device.
 * workspace: device memory of the plan's workspace_bytes, 16-byte aligned.
 * Supported: head_size 64, 128 or 256; num_heads any multiple of num_kv_heads
 *    (groups above 16 query heads take ceil(G / 16) waves per kv head); block_size a
 *    power of two >= 16; batch <= 65535 (<= 8192 for the balanced schedule).
 * Replaces FlashAttnDecode.forward (flash_attn_decode.py:113-181). */
int fk_paged_decode(void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride,
                    const void* k_cache, const void* v_cache, int kv_dtype,
                    const float* k_scale, const float* v_scale, const int32_t* block_tables,
                    int64_t bt_row_stride, const int32_t* ctx_lens, int64_t batch,
                    int num_heads, int num_kv_heads, int head_size, int block_size,
                    int64_t num_blocks, float scale, int window_left, const float* sinks,
                    int64_t part_tokens, int64_t max_parts, void* workspace,
                    int64_t workspace_bytes, void* stream);

/* The two launches fk_paged_decode makes, exposed so a profiler or benchmark can
 * time them separately.  Same arguments as fk_paged_decode.  The partials launch
 * finishes every sequence it holds whole and writes partials for the rest; the
 * reduce launch merges those partials and writes zero rows for empty sequences. */
int fk_paged_decode_partials(void* out, int64_t out_row_stride, const void* q,
                             int64_t q_row_stride, const void* k_cache, const void* v_cache,
                             int kv_dtype, const float* k_scale, const float* v_scale,
                             const int32_t* block_tables, int64_t bt_row_stride,
                             const int32_t* ctx_lens, int64_t batch, int num_heads,
                             int num_kv_heads, int head_size, int block_size,
                             int64_t num_blocks, float scale, int window_left,
                             const float* sinks, int64_t part_tokens, int64_t max_parts,
                             void* workspace, int64_t workspace_bytes, void* stream);
int fk_paged_decode_reduce(void* out, int64_t out_row_stride, const void* q,
                           int64_t q_row_stride, const void* k_cache, const void* v_cache,
                           int kv_dtype, const float* k_scale, const float* v_scale,
                           const int32_t* block_tables, int64_t bt_row_stride,
                           const int32_t* ctx_lens, int64_t batch, int num_heads,
                           int num_kv_heads, int head_size, int block_size, int64_t num_blocks,
                           float scale, int window_left, const float* sinks,
                           int64_t part_tokens, int64_t max_parts, void* workspace,
                           int64_t workspace_bytes, void* stream);

/* Paged decode attention for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference: it is fk_paged_decode without the workspace argument.  The split-context
 * workspace is a static device array of FK_PAGED_DECODE_NOALLOC_MAX_BYTES that each GPU
 * holds from the library's load until the process ends; its address is resolved on the
 * first call on each device.  Arguments and results as fk_paged_decode (same plan from
 * fk_paged_decode_plan); a plan whose workspace_bytes exceeds the static array is
 * rejected with FK_ERR_WORKSPACE (use fk_paged_decode then).  Nothing is allocated.
 * Every call on one device shares the array: calls that overlap on one device
 * (concurrent streams or host threads) race on it and must be serialised by the caller. */
#define FK_PAGED_DECODE_NOALLOC_MAX_BYTES (64LL << 20)
int fk_paged_decode_noalloc(void* out, int64_t out_row_stride, const void* q,
                            int64_t q_row_stride, const void* k_cache, const void* v_cache,
                            int kv_dtype, const float* k_scale, const float* v_scale,
                            const int32_t* block_tables, int64_t bt_row_stride,
                            const int32_t* ctx_lens, int64_t batch, int num_heads,
                            int num_kv_heads, int head_size, int block_size, int64_t num_blocks,
                            float scale, int window_left, const float* sinks,
                            int64_t part_tokens, int64_t max_parts, void* stream);

/* store_kvcache into a cache of another dtype (StoreKVCache.forward with, e.g., a bf16
 * key and a float8_e4m3fn cache: the Triton store converts with tl.store's implicit
 * cast, store_kvcache.py:32-35).  Each element is widened to fp32 and converted to the
 * cache dtype: bf16 / fp16 round to nearest even; fp8 e4m3fn rounds to nearest even,
 * saturates |x| >= 448 to +-448 and keeps NaN.  src_dtype: F32, F16 or BF16;
 * cache_dtype: F32, F16, BF16 or FP8_E4M3FN.  Other arguments as fk_store_kvcache
 * (strides in key/value elements; slots < 0 or >= num_slots are skipped). */
int fk_store_kvcache_convert(const void* key, int64_t key_row_stride, const void* value,
                             int64_t value_row_stride, int src_dtype, void* k_cache,
                             void* v_cache, int cache_dtype, const void* slot_mapping,
                             int slot_is_i64, int64_t tokens, int64_t row_elems,
                             int64_t num_slots, void* stream);

/* Paged prefill attention: FlashAttnPrefill.forward with a block table
 * (fastkernels/tasks/baseline/L1/flash_attn_prefill.py:28-74), the prefill half of
 * Attention._forward_mixed (attention_impl.py:682-731).
 * Sequence b owns query rows [cu_seqlens_q[b], cu_seqlens_q[b+1]) of q / out
 * ([rows, Hq*head_size] bf16, row strides in elements) and the first
 * k_len = cu_seqlens_k[b+1] - cu_seqlens_k[b] tokens of its paged cache (block_tables
 * row b, layout as fk_paged_decode).  Query j of a chunk of q_len sees keys
 * [0, k_len - q_len + j] (causal, aligned to the end); a query with no visible key gets
 * zeros.  causal = 0 lets every query see all k_len keys (flash_attn causal=False).
 * window_left >= 0 (causal only; flash-attn window_size = (window_left, 0)) limits
 * query j to keys [k_len - q_len + j - window_left, k_len - q_len + j]; -1 = no window.
 * sinks: NULL or device fp32 [num_heads] attention-sink logits (s_aux), joining each
 * row's softmax denominator as in fk_paged_decode.
 * max_seqlen_q bounds every chunk (it sizes the grid; at most 65535 blocks of 32
 * query tokens, 128 for GQA group 1).  max_seqlen_k (flash_attn_varlen_func's
 * max_seqlen_k): a bound on every sequence's key count, or 0 if unknown; it only
 * chooses the launch shape (with few query blocks, each block's keys are split over
 * two halves of a work-group and merged).  num_heads any multiple of num_kv_heads.
 * Head sizes: head_size (query / key) and head_size_v (value; out rows are
 * [rows, Hq*head_size_v], the v cache [num_blocks, block_size, Hk, head_size_v]):
 * equal sizes 32, 64, 72, 80, 96, 128 or 256, or 192 / 128 (MLA); others give
 * FK_ERR_UNSUPPORTED.  kv dtype bf16, or fp8 e4m3fn at equal sizes 64, 128, 256 (with
 * k_scale / v_scale as in fk_paged_decode).  A page of key / value rows
 * (block_size * Hk * head size elements) must span fewer than 2^32 bytes (the kernel
 * addresses a page's rows by 32-bit offsets; else FK_ERR_INVALID_ARG).  A -1 (or
 * out-of-range) block-table entry inside a sequence's pages masks that page's keys.
 * No workspace; nothing is allocated.
 * Changed in version 20000: head_size_v added. */
int fk_paged_prefill(void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride,
                     const void* k_cache, const void* v_cache, int kv_dtype, const float* k_scale,
                     const float* v_scale, const int32_t* block_tables, int64_t bt_row_stride,
                     const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t batch,
                     int64_t max_seqlen_q, int64_t max_seqlen_k, int num_heads,
                     int num_kv_heads, int head_size, int head_size_v, int block_size,
                     int64_t num_blocks, float scale, int causal, int window_left,
                     const float* sinks, void* stream);

/* The same attention over dense keys: FlashAttnPrefill.forward without a block table
 * (flash_attn_prefill.py:65-74; Attention._prefill_torch_from_tensors,
 * attention_impl.py:624-638).  key / value: [total_k, Hk*head_size] bf16 rows (strides in
 * elements; views of the qkv buffer allowed); sequence b's keys are rows
 * [cu_seqlens_k[b], cu_seqlens_k[b+1]); value rows are [total_k, Hk*head_size_v].
 * Also FlashAttnVarlen.forward (flash_attn_varlen.py:21-47), including MLA's query /
 * key 192 with value 128 and return_softmax_lse:
 * lse: NULL, or device fp32 [num_heads, lse_row_stride] receiving each row's softmax
 * log-sum-exp at [hq, cu_seqlens_q[b] + j]: ln(sum over visible keys of
 * e^(scale q.k)) (summed in fp32), plus e^sink when sinks are given, -inf for a row
 * with no visible key (flash-attn writes +inf there; fk_merge_attn_states reads
 * both as an empty row).  max_seqlen_k, window_left, sinks and head sizes as
 * fk_paged_prefill.
 * Changed in version 20000: head_size_v, lse and lse_row_stride added. */
int fk_varlen_prefill(void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride,
                      const void* key, int64_t key_row_stride, const void* value,
                      int64_t value_row_stride, const int32_t* cu_seqlens_q,
                      const int32_t* cu_seqlens_k, int64_t batch, int64_t max_seqlen_q,
                      int64_t max_seqlen_k, int num_heads, int num_kv_heads, int head_size,
                      int head_size_v, float scale, int causal, int window_left,
                      const float* sinks, float* lse, int64_t lse_row_stride, void* stream);

/* Work-group key split of the prefill launches (no counterpart in the reference's
 * interface: FlashAttnPrefill / FlashAttnVarlen call flash-attn, whose own split-KV
 * path plays this part).  When a launch would leave CUs without a work-group (one
 * prompt over a few kv heads, or a short chunk over a long cache), each query block's
 * keys are divided over up to 8 work-groups, which leave their partial (O, max, sum)
 * in a caller-owned workspace, and a second kernel merges them with the log-sum-exp
 * rule and writes the rows (and the log-sum-exp).
 * fk_prefill_split_plan: *workspace_bytes = the workspace fk_paged_prefill_ws /
 * fk_varlen_prefill_ws need for these sizes (paged: 1 for the paged entry point,
 * kv_dtype its cache dtype; total_q = rows of q and out, >= cu_seqlens_q[batch]);
 * 0 when the launch does not split (any workspace, or NULL, then gives the plain
 * launch).  The decision uses these host-side bounds only. */
int fk_prefill_split_plan(int paged, int kv_dtype, int64_t batch, int64_t total_q,
                          int64_t max_seqlen_q, int64_t max_seqlen_k, int num_heads,
                          int num_kv_heads, int head_size, int head_size_v, int causal,
                          int64_t* workspace_bytes);

/* fk_paged_prefill / fk_varlen_prefill with the work-group key split's workspace:
 * workspace NULL runs exactly the entry point without _ws; otherwise
 * workspace_bytes must be at least fk_prefill_split_plan's figure for the same
 * arguments (else FK_ERR_WORKSPACE) and the workspace 16-byte aligned.  Its contents
 * need no initialisation and are scratch after the call; calls that share a
 * workspace must be ordered (the same stream).  Results match the entry point
 * without _ws to rounding (each part's O is kept in bf16 before the division by its
 * sum, its max and sums in fp32, and merged in fp32). */
int fk_paged_prefill_ws(void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride,
                        const void* k_cache, const void* v_cache, int kv_dtype,
                        const float* k_scale, const float* v_scale, const int32_t* block_tables,
                        int64_t bt_row_stride, const int32_t* cu_seqlens_q,
                        const int32_t* cu_seqlens_k, int64_t batch, int64_t max_seqlen_q,
                        int64_t max_seqlen_k, int num_heads, int num_kv_heads, int head_size,
                        int head_size_v, int block_size, int64_t num_blocks, float scale,
                        int causal, int window_left, const float* sinks, int64_t total_q,
                        void* workspace, int64_t workspace_bytes, void* stream);
int fk_varlen_prefill_ws(void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride,
                         const void* key, int64_t key_row_stride, const void* value,
                         int64_t value_row_stride, const int32_t* cu_seqlens_q,
                         const int32_t* cu_seqlens_k, int64_t batch, int64_t max_seqlen_q,
                         int64_t max_seqlen_k, int num_heads, int num_kv_heads, int head_size,
                         int head_size_v, float scale, int causal, int window_left,
                         const float* sinks, float* lse, int64_t lse_row_stride,
                         int64_t total_q, void* workspace, int64_t workspace_bytes,
                         void* stream);

/* Per-head q/k RMSNorm (optional) + rotary embedding + store_kvcache in one launch:
 * the attention block between the qkv projection and the decode
 * (fastkernels/tasks/baseline/L2/attention.py:120-140: q_norm / k_norm on [N, H, D]
 * views, then rotary_emb; then attention_impl.py:323-325 store_kvcache).
 * query [tokens, Hq*D], key / value [tokens, Hk*D]: rows with the given strides (views
 * of the fused qkv buffer), heads contiguous.  query and key are rewritten in place
 * (normed when q_weight / k_weight are given, both or neither, [D] of the dtype; then
 * rotated as fk_rotary_embedding); the rotated key rows and the value rows go to
 * cache slot slot_mapping[t] (skipped outside [0, num_slots)).  Caches:
 * [num_slots, Hk, D] of the dtype.  Vector path only: 16-byte aligned rows, caches and
 * weights, D / (16 / elem) a power of two <= 64; otherwise FK_ERR_UNSUPPORTED.  The
 * results are bit-identical to fk_rmsnorm per head row, fk_rotary_embedding and
 * fk_store_kvcache in sequence. */
int fk_qk_norm_rope_store(const int64_t* positions, void* query, int64_t q_row_stride, void* key,
                          int64_t k_row_stride, const void* value, int64_t v_row_stride,
                          const void* q_weight, const void* k_weight, float eps,
                          const void* cos_sin, int cache_dtype, int64_t max_position, int rot_dim,
                          int is_neox, void* k_cache, void* v_cache, const void* slot_mapping,
                          int slot_is_i64, int64_t num_slots, int64_t tokens, int num_heads,
                          int num_kv_heads, int head_size, int dtype, void* stream);

/* store_kvcache + paged decode in one launch (plus the merge launch): the
 * decode step of Attention.forward_impl
 * (fastkernels/tasks/baseline/L2/attention_impl.py:313-363, :436-450), which calls
 * StoreKVCache (store_kvcache.py:16-35) and then FlashAttnDecode.forward
 * (flash_attn_decode.py:113-181).
 * key/value: [batch, Hk, head_size] of the cache element type (bf16 or fp8 e4m3fn),
 * row strides in elements, 16-byte aligned.  slot_mapping: int32 or int64 [batch];
 * negative or out-of-range entries are not stored.  All other arguments as
 * fk_paged_decode (same plan and workspace).
 * Decode-step layout: slot_mapping[b] is the slot of position ctx_lens[b] - 1 in
 * block_tables[b] (engine.py:5020-5024).  Then the cache and the output equal
 * fk_store_kvcache followed by fk_paged_decode, bit for bit: the waves that stream
 * that position write the row just before they load it.  A slot that another
 * sequence reads in the same call is written too, but that sequence's output is
 * unspecified. */
int fk_store_paged_decode(void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride,
                          const void* key, int64_t key_row_stride, const void* value,
                          int64_t value_row_stride, const void* slot_mapping, int slot_is_i64,
                          void* k_cache, void* v_cache, int kv_dtype, const float* k_scale,
                          const float* v_scale, const int32_t* block_tables,
                          int64_t bt_row_stride, const int32_t* ctx_lens, int64_t batch,
                          int num_heads, int num_kv_heads, int head_size, int block_size,
                          int64_t num_blocks, float scale, int window_left, const float* sinks,
                          int64_t part_tokens, int64_t max_parts, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* Log-sum-exp merge of two partial attention results (split-KV / prefix+suffix):
 *   out[t,h,:] = (prefix[t,h,:] e^(p - M) + suffix[t,h,:] e^(s - M)) / (e^(p - M) + e^(s - M))
 *   with p = prefix_lse[h,t], s = suffix_lse[h,t] (natural log, +inf read as -inf),
 *   M = max(p, s), out_lse[h,t] = log(e^(p-M) + e^(s-M)) + M; when M = -inf the
 *   prefix rows are copied and out_lse = -inf.  out_lse may be NULL.
 * out/prefix/suffix: [tokens, heads, head_size] with the given token and head strides
 * (prefix and suffix share theirs); lse tensors: fp32 [heads, tokens] contiguous.
 * Tokens >= prefill_tokens_with_context (a negative value = all tokens) copy the
 * suffix and its lse.  dtype: F32, F16 or BF16 (computed in fp32).
 * out_dtype: dtype, or FP8_E4M3FN for an fp8 output (output_scale: device fp32
 * scalar): every output value, merged or copied, becomes
 * e4m3fn(clamp(v * (1 / *output_scale), -448, 448)) (round to nearest even; the
 * clamp takes NaN to 448), as merge_attn_states.cu:2436-2571 with USE_FP8_OUTPUT;
 * out strides are then in bytes.
 * Replaces merge_attn_states / MergeAttnStates.forward
 * (fastkernels/tasks/baseline/L1/merge_attn_states.py:30-122).
 * Changed in version 20000: out_dtype and output_scale added. */
int fk_merge_attn_states(void* out, int64_t out_token_stride, int64_t out_head_stride,
                         float* out_lse, const void* prefix, const float* prefix_lse,
                         const void* suffix, const float* suffix_lse, int64_t in_token_stride,
                         int64_t in_head_stride, int64_t tokens, int heads, int head_size,
                         int64_t prefill_tokens_with_context, int dtype, int out_dtype,
                         const float* output_scale, void* stream);

/* SiLU-and-mul: out[r, j] = cast(cast(silu(x[r, j])) * x[r, d + j]) for j < d.
 * x: [rows, 2d] rows `x_row_stride` elements apart; out: [rows, d] rows
 * `out_row_stride` apart.  dtype F32, F16 or BF16.
 * Replaces _C.silu_and_mul(out, x) (silu_and_mul.py:24-30, silu_and_mul.cu:951-956);
 * the bf16-rounded activation matches forward_native (silu_and_mul.py:19-22). */
int fk_silu_and_mul(void* out, int64_t out_row_stride, const void* x, int64_t x_row_stride,
                    int64_t rows, int64_t d, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FASTKERNELS_AMD_H_ */
