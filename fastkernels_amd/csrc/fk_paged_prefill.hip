// C entry points of the prefill attention kernel (fk_prefill_kernel.h):
// fk_paged_prefill (FlashAttnPrefill with a block table) and fk_varlen_prefill
// (dense keys: FlashAttnPrefill without one, and FlashAttnVarlen).  This file
// instantiates the kernel at D = DV in {64, 128, 256} with bf16 and fp8 pages
// and dense keys; fk_prefill_heads.hip instantiates the other head sizes.
#include <algorithm>

#include "fk_prefill_kernel.h"

namespace fk {
namespace {

// (query / key, value) head sizes the library is built for.
bool prefill_heads_supported(int d, int dv, bool fp8_pages) {
  if (fp8_pages) return d == dv && (d == 64 || d == 128 || d == 256);
  if (d == dv)
    return d == 32 || d == 64 || d == 72 || d == 80 || d == 96 || d == 128 || d == 256;
  return d == 192 && dv == 128;
}

template <int D>
void launch_prefill_d(bool paged, bool fp8, bool split, const PrefillParams& P, dim3 grid,
                      const int32_t* bt, const int32_t* cu_q, const int32_t* cu_k,
                      hipStream_t stream) {
  if (paged && fp8)
    launch_prefill<true, true, D, D>(split, P, grid, bt, cu_q, cu_k, stream);
  else
    launch_prefill_bf16<D, D>(paged, split, P, grid, bt, cu_q, cu_k, stream);
}

int prefill_entry(const char* name, bool paged, void* out, int64_t out_row_stride, const void* q,
                  int64_t q_row_stride, const void* k, int64_t k_row_bytes, const void* v,
                  int64_t v_row_bytes, int kv_dtype, const float* k_scale, const float* v_scale,
                  const int32_t* block_tables, int64_t bt_row_stride,
                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t batch,
                  int64_t max_seqlen_q, int64_t max_seqlen_k, int num_heads, int num_kv_heads,
                  int head_size, int head_size_v, int block_size, int64_t num_blocks,
                  float scale, int causal, int window_left, const float* sinks, float* lse,
                  int64_t lse_row_stride, void* stream) {
  FK_REQUIRE(batch >= 0 && batch <= 65535, "%s: batch %lld out of range [0, 65535]", name,
             (long long)batch);
  FK_REQUIRE(window_left >= -1, "%s: window_left %d must be -1 (no window) or >= 0", name,
             window_left);
  FK_REQUIRE(window_left < 0 || causal,
             "%s: a sliding window needs causal attention (window_size = (left, 0))", name);
  FK_REQUIRE(max_seqlen_q >= 0 && max_seqlen_q <= (int64_t(1) << 30),
             "%s: max_seqlen_q %lld out of range", name, (long long)max_seqlen_q);
  FK_REQUIRE(max_seqlen_k >= 0, "%s: max_seqlen_k %lld must be >= 0 (0: unknown)", name,
             (long long)max_seqlen_k);
  FK_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             "%s: num_heads %d must be a positive multiple of num_kv_heads %d", name, num_heads,
             num_kv_heads);
  if (!prefill_heads_supported(head_size, head_size_v, kv_dtype == FK_DTYPE_FP8_E4M3FN && paged))
    return set_error(FK_ERR_UNSUPPORTED,
                     "%s: head sizes (query/key %d, value %d) unsupported: equal sizes 32, 64, 72, "
                     "80, 96, 128 or 256, or 192 / 128 (fp8 pages: 64, 128 or 256)",
                     name, head_size, head_size_v);
  FK_REQUIRE(num_kv_heads <= 32767, "%s: too many kv heads", name);
  if (paged) {
    FK_REQUIRE(block_size >= kTile && (block_size & (block_size - 1)) == 0,
               "%s: block_size %d must be a power of two >= 16", name, block_size);
    FK_REQUIRE(kv_dtype == FK_DTYPE_BF16 || kv_dtype == FK_DTYPE_FP8_E4M3FN,
               "%s: kv dtype %d unsupported (bf16 or fp8 e4m3fn)", name, kv_dtype);
  }
  FK_REQUIRE(q_row_stride >= static_cast<int64_t>(num_heads) * head_size &&
                 out_row_stride >= static_cast<int64_t>(num_heads) * head_size_v,
             "%s: row stride shorter than num_heads * head_size", name);
  const int64_t elem = kv_dtype == FK_DTYPE_FP8_E4M3FN ? 1 : 2;
  FK_REQUIRE(k_row_bytes >= num_kv_heads * head_size * elem &&
                 v_row_bytes >= num_kv_heads * head_size_v * elem,
             "%s: key/value rows shorter than num_kv_heads * head size", name);
  FK_REQUIRE(!lse || lse_row_stride >= 0, "%s: lse row stride must be >= 0", name);
  FK_REQUIRE(!lse || !paged, "%s: the log-sum-exp output is built for dense keys only", name);
  if (batch == 0 || max_seqlen_q == 0) return FK_OK;
  FK_REQUIRE(out && q && k && v && cu_seqlens_q && cu_seqlens_k && (!paged || block_tables),
             "%s: null pointer", name);
  FK_REQUIRE(!paged || num_blocks >= 1, "%s: the cache must hold at least one block", name);
  FK_REQUIRE(aligned16(q) && aligned16(out) && aligned16(k) && aligned16(v) &&
                 q_row_stride % 8 == 0 && out_row_stride % 8 == 0 && k_row_bytes % 16 == 0 &&
                 v_row_bytes % 16 == 0,
             "%s: q/out/keys/values must be 16-byte aligned with 16-byte row strides", name);
  const int gqa = num_heads / num_kv_heads;
  const int hw = gqa < kPrefillWaves ? gqa : kPrefillWaves;  // query heads per work-group
  const int64_t wg_tokens =
      static_cast<int64_t>(kPrefillWaves / hw) * 16 * col_blocks_for(head_size, head_size_v);
  const int64_t qblocks = (max_seqlen_q + wg_tokens - 1) / wg_tokens;
  PrefillParams P;
  P.out = static_cast<uint16_t*>(out);
  P.out_row_stride = out_row_stride;
  P.q = static_cast<const uint16_t*>(q);
  P.q_row_stride = q_row_stride;
  P.k_cache = static_cast<const uint8_t*>(k);
  P.v_cache = static_cast<const uint8_t*>(v);
  P.k_row_bytes = k_row_bytes;
  P.v_row_bytes = v_row_bytes;
  P.k_scale = k_scale;
  P.v_scale = v_scale;
  P.bt_row_stride = paged ? bt_row_stride : 0;
  P.num_kv_heads = num_kv_heads;
  P.gqa = num_heads / num_kv_heads;
  P.block_size_log2 = paged ? __builtin_ctz(static_cast<unsigned>(block_size)) : 0;
  P.num_blocks = paged ? num_blocks : 0;
  FK_REQUIRE(scale > 0.f && scale < __builtin_huge_valf(),
             "%s: softmax scale must be positive and finite (got %g)", name, (double)scale);
  P.scale_log2 = scale * kLog2e;
  P.causal = causal ? 1 : 0;
  P.window_left = window_left;
  P.sinks = sinks;
  P.lse = lse;
  P.lse_row_stride = lse_row_stride;
  const int hsplit = (gqa + hw - 1) / hw;
  FK_REQUIRE(qblocks <= 65535, "%s: max_seqlen_q %lld needs more than 65535 query blocks", name,
             (long long)max_seqlen_q);
  const dim3 grid(static_cast<unsigned>(num_kv_heads * hsplit), static_cast<unsigned>(batch),
                  static_cast<unsigned>(qblocks));
  hipStream_t s = as_stream(stream);
  const bool fp8 = kv_dtype == FK_DTYPE_FP8_E4M3FN;
  // Key split when the grid (before pairing) holds at most two 4-wave
  // work-groups per CU: pairing then leaves at most one, so one wave per SIMD.
  // Key split when the 4-wave launch would leave SIMDs with one wave: fewer
  // work-groups than two per CU.  A causal sequence with fewer cached keys than
  // twice its queries pairs its blocks two per work-group; max_seqlen_k (a
  // bound on every sequence's keys, 0 = unknown) tells whether that can happen.
  const bool may_pair = causal && max_seqlen_k > 0 && max_seqlen_k < 2 * max_seqlen_q;
  const int64_t wgs = static_cast<int64_t>(num_kv_heads) * hsplit * batch *
                      (may_pair ? (qblocks + 1) / 2 : qblocks);
  const bool split = (std::max(head_size, head_size_v) <= 192 || paged) &&
                     wgs < 2LL * num_cus();
  if (head_size == head_size_v && (head_size == 64 || head_size == 128 || head_size == 256)) {
    switch (head_size) {
      case 64: launch_prefill_d<64>(paged, fp8, split, P, grid, block_tables, cu_seqlens_q, cu_seqlens_k, s); break;
      case 256: launch_prefill_d<256>(paged, fp8, split, P, grid, block_tables, cu_seqlens_q, cu_seqlens_k, s); break;
      default: launch_prefill_d<128>(paged, fp8, split, P, grid, block_tables, cu_seqlens_q, cu_seqlens_k, s); break;
    }
  } else if (!launch_prefill_extra(head_size, head_size_v, paged, split, P, grid, block_tables,
                                   cu_seqlens_q, cu_seqlens_k, s)) {
    return set_error(FK_ERR_UNSUPPORTED, "%s: head sizes %d / %d not built", name, head_size,
                     head_size_v);
  }
  return check_launch(name);
}

}  // namespace
}  // namespace fk

extern "C" int fk_paged_prefill(void* out, int64_t out_row_stride, const void* q,
                                int64_t q_row_stride, const void* k_cache, const void* v_cache,
                                int kv_dtype, const float* k_scale, const float* v_scale,
                                const int32_t* block_tables, int64_t bt_row_stride,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                int64_t batch, int64_t max_seqlen_q, int64_t max_seqlen_k,
                                int num_heads, int num_kv_heads, int head_size, int head_size_v,
                                int block_size, int64_t num_blocks, float scale, int causal,
                                int window_left, const float* sinks, void* stream) {
  const int64_t elem = kv_dtype == FK_DTYPE_FP8_E4M3FN ? 1 : 2;
  const int64_t k_row = static_cast<int64_t>(num_kv_heads) * head_size * elem;
  const int64_t v_row = static_cast<int64_t>(num_kv_heads) * head_size_v * elem;
  return fk::prefill_entry("fk_paged_prefill", true, out, out_row_stride, q, q_row_stride,
                           k_cache, k_row, v_cache, v_row, kv_dtype, k_scale, v_scale,
                           block_tables, bt_row_stride, cu_seqlens_q, cu_seqlens_k, batch,
                           max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_size,
                           head_size_v, block_size, num_blocks, scale, causal, window_left,
                           sinks, nullptr, 0, stream);
}

extern "C" int fk_varlen_prefill(void* out, int64_t out_row_stride, const void* q,
                                 int64_t q_row_stride, const void* key, int64_t key_row_stride,
                                 const void* value, int64_t value_row_stride,
                                 const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                 int64_t batch, int64_t max_seqlen_q, int64_t max_seqlen_k,
                                 int num_heads, int num_kv_heads, int head_size, int head_size_v,
                                 float scale, int causal, int window_left, const float* sinks,
                                 float* lse, int64_t lse_row_stride, void* stream) {
  return fk::prefill_entry("fk_varlen_prefill", false, out, out_row_stride, q, q_row_stride, key,
                           key_row_stride * 2, value, value_row_stride * 2, FK_DTYPE_BF16,
                           nullptr, nullptr, nullptr, 0, cu_seqlens_q, cu_seqlens_k, batch,
                           max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_size,
                           head_size_v, 16, 0, scale, causal, window_left, sinks, lse,
                           lse_row_stride, stream);
}
