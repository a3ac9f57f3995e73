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

// Launch shape of a prefill call, from the host-side bounds alone (the plan
// entry point and the launch agree on it).
struct PrefillShape {
  int64_t qblocks;  // query blocks per sequence (grid z before the key parts)
  int hsplit;       // work-groups per kv head (head groups of up to 4)
  int ks;           // key parts within a work-group (1 or 2)
  int xs;           // key parts over work-groups (1: none), with a workspace
  int ks_plain;     // ks of the same call without a workspace (xs = 1)
};

PrefillShape prefill_shape(bool paged, bool fp8, int64_t batch, int64_t max_seqlen_q,
                           int64_t max_seqlen_k, int num_heads, int num_kv_heads, int head_size,
                           int head_size_v, int causal) {
  PrefillShape sh;
  const int gqa = num_heads / num_kv_heads;
  const int hw = gqa < kPrefillWaves ? gqa : kPrefillWaves;  // query heads per work-group
  const int64_t wg_tokens =
      static_cast<int64_t>(kPrefillWaves / hw) * 16 * col_blocks_for(head_size, head_size_v);
  sh.qblocks = (max_seqlen_q + wg_tokens - 1) / wg_tokens;
  sh.hsplit = (gqa + hw - 1) / hw;
  // Key split when the 4-wave launch would leave SIMDs with one wave: fewer
  // work-groups than two per CU.  A causal sequence with fewer cached keys than
  // twice its queries pairs its blocks two per work-group; max_seqlen_k (a
  // bound on every sequence's keys, 0 = unknown) tells whether that can happen.
  const bool may_pair = causal && max_seqlen_k > 0 && max_seqlen_k < 2 * max_seqlen_q;
  const int64_t wgs = static_cast<int64_t>(num_kv_heads) * sh.hsplit * batch *
                      (may_pair ? (sh.qblocks + 1) / 2 : sh.qblocks);
  sh.ks = ((std::max(head_size, head_size_v) <= 192 || paged) && wgs < 2LL * num_cus()) ? 2 : 1;
  sh.ks_plain = sh.ks;
  sh.xs = 1;
  const int64_t ncu = num_cus();
  // Where the key split would run (fewer 4-wave work-groups than two per CU):
  // 4-wave work-groups, two per CU, with each block's keys in xs parts over
  // work-groups, instead of one 8-wave key-split work-group per block, for
  // chunks over cached keys (blocks not paired) and, at head sizes up to 64 with
  // bf16 pages, for causal pairs.  xs = floor(2 CUs / work-groups) when that is
  // at least 2 and fills 7/8 of the two-per-CU slots, else the ceiling (at most
  // kMaxKeyParts), and only while a part keeps at least 20 stages of 32 keys (40
  // above head size 64: a dense 2048-token non-causal prompt at 16 / 16 / 80
  // heads, 2 parts of 32 stages, went 48.8 -> 52.9).
  // Measured on MI355X (whole call, µs, key split -> this; same box, A/B in
  // alternating processes, two rounds averaged): Qwen3-8B heads (32 / 8 / 128)
  // 1x512 over 8192 102.9 -> 91.2, 2x512 over 4096 92.8 -> 86.5, 3x512 over 4096
  // 160.2 -> 145.9, fp8 pages 1x512 over 8192 114.7 -> 109.8; Qwen3-Next heads
  // (16 / 2 / 256) 1x512 over 8192 116.0 -> 106.4, 2x512 over 4096 109.4 ->
  // 103.5; Whisper heads (20 / 20 / 64) 4x512 over 4096 112.9 -> 80.4, 2x512
  // over 4096 57.2 -> 47.8, 1x512 over 8192 54.9 -> 48.5, prompts 1x2048 45.2 ->
  // 40.8, 2x2048 80.5 -> 61.7, 1x4096 132.0 -> 93.7; dense keys, 1x512 over 8192
  // at Qwen3-8B heads 98.6 -> 90.1 and at MLA's (16 / 16 / 192 / 128, not
  // causal) 92.7 -> 81.2, 2x512 over 4096 93.7 -> 89.4.  In single probes, causal
  // pairs at head 128 and 256 were slower this way (1x2048: 58.9 -> 68.3 and
  // 65.7 -> 73.8; they keep the key split with split pairs), and so were short
  // parts (Whisper heads 2x1024 at 3 parts of 12 stages: 31.6 -> 33.2).
  if (sh.ks == 2 && wgs > 0 &&
      (!may_pair || (!fp8 && std::max(head_size, head_size_v) <= 64))) {
    const int64_t slots = 2 * ncu;
    int64_t xs = slots / wgs;
    if (xs < 2 || 8 * wgs * xs < 7 * slots) xs = (slots + wgs - 1) / wgs;
    xs = std::min<int64_t>(xs, kMaxKeyParts);
    const double stages = static_cast<double>(std::max(max_seqlen_k, max_seqlen_q) +
                                              (may_pair ? wg_tokens : 0)) /
                          kStageKeys;  // the heaviest work-group's stages (a pair's)
    const double min_stages = std::max(head_size, head_size_v) <= 64 ? 20.0 : 40.0;
    if (xs >= 2 && stages >= min_stages * xs && sh.qblocks * xs <= 65535) {
      sh.ks = 1;
      sh.xs = static_cast<int>(xs);
      return sh;
    }
  }
  // Otherwise, work-group key split when even the key split leaves CUs without
  // a work-group (one work-group per CU at this size): each block's keys in xs
  // parts over xs work-groups, merged by prefill_merge_kernel.  xs minimises an
  // estimate of the call's time (µs; constants measured on MI355X): the heaviest work-group
  // streams S stages of 32 keys (all of max_seqlen_k; a causal pair of blocks
  // about max_seqlen_k plus one block) at kStageUs per stage and key-split half,
  // plus kBlockUs per block (its queries, the first stage's latency, the rows);
  // the work-groups run ceil(wgs * xs / CUs) rounds; the parts' states are
  // written and read back at kMergeBytesPerUs, plus kMergeUs for the merge's
  // launch.  Short blocks (prompts) keep one part: their per-block costs stay.
  // (The constants were fitted with the parts' O in fp32; the estimate keeps
  // those bytes, so that its choices stay the measured ones.)
  if (wgs > 0 && wgs < ncu) {
    constexpr double kStageUs = 1.2, kBlockUs = 6.0, kMergeUs = 3.0;
    constexpr double kMergeBytesPerUs = 2.5e6;
    const int64_t keys = std::max(max_seqlen_k, max_seqlen_q);
    const int blocks = may_pair ? 2 : 1;
    const double S = static_cast<double>(keys + (may_pair ? wg_tokens : 0)) / kStageKeys;
    const double row_bytes =
        static_cast<double>(batch) * max_seqlen_q * num_heads * (head_size_v + kPartMl) * 4;
    double best = S / sh.ks * kStageUs + blocks * kBlockUs;
    for (int xs = 2; xs <= kMaxKeyParts; ++xs) {
      if (S < 4.0 * xs * sh.ks || sh.qblocks * xs > 65535) break;
      const double rounds = static_cast<double>((wgs * xs + ncu - 1) / ncu);
      const double t = rounds * (S / (sh.ks * xs) * kStageUs + blocks * kBlockUs) +
                       xs * row_bytes / kMergeBytesPerUs + kMergeUs;
      if (t < best) {
        best = t;
        sh.xs = xs;
      }
    }
  }
  return sh;
}

// Bytes of the work-group key split's partial states (0 without the split).
int64_t prefill_ws_bytes(const PrefillShape& sh, int64_t total_q, int num_heads, int head_size_v) {
  if (sh.xs <= 1) return 0;
  const int64_t bytes = part_ml_offset(sh.xs, total_q, num_heads, head_size_v) +
                        static_cast<int64_t>(sh.xs) * total_q * num_heads * kPartMl * 4;
  return (bytes + 255) / 256 * 256;
}

// The merge of a work-group key split: per (row, head), the parts' states
// combined with the log-sum-exp rule (M = max m_p, O = sum O_p 2^(m_p - M),
// l = sum l_p 2^(m_p - M); a part that saw no key has m_p = -inf and weighs 0),
// the sink joined to the sum, O / l written as bf16 (0 for a row with no visible
// key), and the log-sum-exp from the fp32 sums.  A thread takes 8 dims of one
// (row, head); rows past cu_seqlens_q[batch] are left alone.
struct PrefillMergeParams {
  uint16_t* out;
  int64_t out_row_stride;
  const void* part;
  int64_t part_rows;
  int xs;
  int num_heads;
  int dv;
  const int32_t* cu_q;
  int64_t batch;
  const float* sinks;
  float* lse;
  int64_t lse_row_stride;
};

__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillMergeParams M) {
  const int chunks = M.dv / 8;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t rh = t / chunks;
  const int c8 = static_cast<int>(t - rh * chunks);
  const int64_t rows = M.cu_q[M.batch];
  if (rh >= rows * M.num_heads) return;
  const int64_t row = rh / M.num_heads;
  const int hq = static_cast<int>(rh - row * M.num_heads);
  const int64_t plane = M.part_rows * M.num_heads;  // (row, head) records per part
  const float* const ml = reinterpret_cast<const float*>(
      static_cast<const uint8_t*>(M.part) + part_ml_offset(M.xs, M.part_rows, M.num_heads, M.dv));
  const uint16_t* const po = static_cast<const uint16_t*>(M.part);
  // Every part's record and O slice (8 bf16) are loaded before any is used.
  float4 rec[kMaxKeyParts];
  uint4 ov[kMaxKeyParts];
#pragma unroll
  for (int p = 0; p < kMaxKeyParts; ++p) {
    if (p < M.xs) {
      rec[p] = *reinterpret_cast<const float4*>(ml + (p * plane + rh) * kPartMl);
      ov[p] = *reinterpret_cast<const uint4*>(po + (p * plane + rh) * M.dv + 8 * c8);
    }
  }
  float mx = kNegInf;
#pragma unroll
  for (int p = 0; p < kMaxKeyParts; ++p)
    if (p < M.xs) mx = fmaxf(mx, rec[p].x);
  float l = 0.f, l32 = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int p = 0; p < kMaxKeyParts; ++p) {
    if (p < M.xs) {
      const float w = rec[p].x == kNegInf ? 0.f : __builtin_amdgcn_exp2f(rec[p].x - mx);
      l += w * rec[p].y;
      l32 += w * rec[p].z;
      const uint32_t ow[4] = {ov[p].x, ov[p].y, ov[p].z, ov[p].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // dims 2i (low half) and 2i + 1 (high half)
        acc[2 * i] += w * __builtin_bit_cast(float, ow[i] << 16);
        acc[2 * i + 1] += w * __builtin_bit_cast(float, ow[i] & 0xffff0000u);
      }
    }
  }
  const float sink2 = M.sinks ? M.sinks[hq] * kLog2e : kNegInf;
  l = with_sink(l, mx, sink2);
  const float f = l > 0.f ? 1.f / l : 0.f;
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bf16x2_t pk = {static_cast<__bf16>(acc[2 * i] * f), static_cast<__bf16>(acc[2 * i + 1] * f)};
    w[i] = __builtin_bit_cast(uint32_t, pk);
  }
  *reinterpret_cast<uint4*>(M.out + row * M.out_row_stride + static_cast<int64_t>(hq) * M.dv +
                            8 * c8) = make_uint4(w[0], w[1], w[2], w[3]);
  if (M.lse && c8 == 0) {
    l32 = with_sink(l32, mx, sink2);
    M.lse[hq * M.lse_row_stride + row] =
        l32 > 0.f ? (mx + __log2f(l32)) * 0.6931471805599453f : kNegInf;
  }
}

int prefill_entry(const char* name, bool paged, void* out, int64_t out_row_stride, const void* q,
                  int64_t q_row_stride, const void* k, int64_t k_row_bytes, const void* v,
                  int64_t v_row_bytes, int kv_dtype, const float* k_scale, const float* v_scale,
                  const int32_t* block_tables, int64_t bt_row_stride,
                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t batch,
                  int64_t max_seqlen_q, int64_t max_seqlen_k, int num_heads, int num_kv_heads,
                  int head_size, int head_size_v, int block_size, int64_t num_blocks,
                  float scale, int causal, int window_left, const float* sinks, float* lse,
                  int64_t lse_row_stride, int64_t total_q, void* workspace, int64_t ws_bytes,
                  void* stream) {
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
  // The kernel addresses a page's rows (a dense tile's 16 rows) by 32-bit offsets
  // from the page's (tile's) first row.
  FK_REQUIRE((paged ? static_cast<int64_t>(block_size) : int64_t(kTile)) *
                     (k_row_bytes > v_row_bytes ? k_row_bytes : v_row_bytes) <=
                 (int64_t(1) << 32) - 1,
             "%s: a page of key/value rows must span fewer than 2^32 bytes", name);
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
  const bool fp8 = kv_dtype == FK_DTYPE_FP8_E4M3FN;
  PrefillShape sh = prefill_shape(paged, fp8, batch, max_seqlen_q, max_seqlen_k, num_heads,
                                  num_kv_heads, head_size, head_size_v, causal);
  if (workspace == nullptr) {
    sh.xs = 1;  // no workspace: the launch without the work-group key split
    sh.ks = sh.ks_plain;
  } else {
    FK_REQUIRE(total_q >= 0, "%s: total_q %lld must be >= 0", name, (long long)total_q);
    const int64_t need = prefill_ws_bytes(sh, total_q, num_heads, head_size_v);
    if (ws_bytes < need)
      return set_error(FK_ERR_WORKSPACE, "%s: workspace of %lld bytes < %lld required", name,
                       (long long)ws_bytes, (long long)need);
    FK_REQUIRE(aligned16(workspace), "%s: workspace must be 16-byte aligned", name);
  }
  const int64_t qblocks = sh.qblocks;
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
  P.xs = sh.xs;
  P.part = workspace;
  P.part_rows = total_q;
  P.num_heads = num_heads;
  FK_REQUIRE(qblocks <= 65535, "%s: max_seqlen_q %lld needs more than 65535 query blocks", name,
             (long long)max_seqlen_q);
  const dim3 grid(static_cast<unsigned>(num_kv_heads * sh.hsplit), static_cast<unsigned>(batch),
                  static_cast<unsigned>(qblocks * sh.xs));
  hipStream_t s = as_stream(stream);
  const bool split = sh.ks > 1;
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
  if (sh.xs > 1) {
    PrefillMergeParams M;
    M.out = static_cast<uint16_t*>(out);
    M.out_row_stride = out_row_stride;
    M.part = P.part;
    M.part_rows = total_q;
    M.xs = sh.xs;
    M.num_heads = num_heads;
    M.dv = head_size_v;
    M.cu_q = cu_seqlens_q;
    M.batch = batch;
    M.sinks = sinks;
    M.lse = lse;
    M.lse_row_stride = lse_row_stride;
    const int64_t threads = total_q * num_heads * (head_size_v / 8);
    if (threads > 0)
      hipLaunchKernelGGL(prefill_merge_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)),
                         dim3(256), 0, s, M);
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
                           sinks, nullptr, 0, 0, nullptr, 0, stream);
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
                           lse_row_stride, 0, nullptr, 0, stream);
}

extern "C" int fk_prefill_split_plan(int paged, int kv_dtype, int64_t batch, int64_t total_q,
                                     int64_t max_seqlen_q, int64_t max_seqlen_k, int num_heads,
                                     int num_kv_heads, int head_size, int head_size_v,
                                     int causal, int64_t* workspace_bytes) {
  const char* name = "fk_prefill_split_plan";
  FK_REQUIRE(workspace_bytes != nullptr, "%s: null workspace_bytes", name);
  *workspace_bytes = 0;
  FK_REQUIRE(batch >= 0 && total_q >= 0 && max_seqlen_q >= 0 && max_seqlen_k >= 0,
             "%s: negative size", name);
  FK_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             "%s: num_heads %d must be a positive multiple of num_kv_heads %d", name, num_heads,
             num_kv_heads);
  if (batch == 0 || max_seqlen_q == 0 || total_q == 0) return FK_OK;
  const fk::PrefillShape sh =
      fk::prefill_shape(paged != 0, kv_dtype == FK_DTYPE_FP8_E4M3FN, batch, max_seqlen_q,
                        max_seqlen_k, num_heads, num_kv_heads, head_size, head_size_v, causal);
  *workspace_bytes = fk::prefill_ws_bytes(sh, total_q, num_heads, head_size_v);
  return FK_OK;
}

extern "C" int fk_paged_prefill_ws(void* out, int64_t out_row_stride, const void* q,
                                   int64_t q_row_stride, const void* k_cache, const void* v_cache,
                                   int kv_dtype, const float* k_scale, const float* v_scale,
                                   const int32_t* block_tables, int64_t bt_row_stride,
                                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                   int64_t batch, int64_t max_seqlen_q, int64_t max_seqlen_k,
                                   int num_heads, int num_kv_heads, int head_size,
                                   int head_size_v, int block_size, int64_t num_blocks,
                                   float scale, int causal, int window_left, const float* sinks,
                                   int64_t total_q, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  const int64_t elem = kv_dtype == FK_DTYPE_FP8_E4M3FN ? 1 : 2;
  const int64_t k_row = static_cast<int64_t>(num_kv_heads) * head_size * elem;
  const int64_t v_row = static_cast<int64_t>(num_kv_heads) * head_size_v * elem;
  return fk::prefill_entry("fk_paged_prefill_ws", true, out, out_row_stride, q, q_row_stride,
                           k_cache, k_row, v_cache, v_row, kv_dtype, k_scale, v_scale,
                           block_tables, bt_row_stride, cu_seqlens_q, cu_seqlens_k, batch,
                           max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_size,
                           head_size_v, block_size, num_blocks, scale, causal, window_left,
                           sinks, nullptr, 0, total_q, workspace, workspace_bytes, stream);
}

extern "C" int fk_varlen_prefill_ws(void* out, int64_t out_row_stride, const void* q,
                                    int64_t q_row_stride, const void* key, int64_t key_row_stride,
                                    const void* value, int64_t value_row_stride,
                                    const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                    int64_t batch, int64_t max_seqlen_q, int64_t max_seqlen_k,
                                    int num_heads, int num_kv_heads, int head_size,
                                    int head_size_v, float scale, int causal, int window_left,
                                    const float* sinks, float* lse, int64_t lse_row_stride,
                                    int64_t total_q, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  return fk::prefill_entry("fk_varlen_prefill_ws", false, out, out_row_stride, q, q_row_stride,
                           key, key_row_stride * 2, value, value_row_stride * 2, FK_DTYPE_BF16,
                           nullptr, nullptr, nullptr, 0, cu_seqlens_q, cu_seqlens_k, batch,
                           max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_size,
                           head_size_v, 16, 0, scale, causal, window_left, sinks, lse,
                           lse_row_stride, total_q, workspace, workspace_bytes, stream);
}
