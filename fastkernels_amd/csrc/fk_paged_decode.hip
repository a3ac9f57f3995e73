// Paged decode attention for MI355X (gfx950): split-context ("flash-decoding")
// with GQA-packed MFMA tiles and a length-balanced schedule.
//
// Semantics (one query token per sequence, at position ctx_lens[b] - 1):
//   out[b, hq] = sum_t softmax_t(scale * q[b,hq] . K[b,t]) V[b,t],  lo_b <= t < ctx_lens[b]
// with lo_b = 0, or ctx_lens[b] - 1 - window_left under a sliding window
// (window_size = (window_left, 0): keys [q_pos - window_left, q_pos], the
// SLIDING_WINDOW = 1 + window_size[0] mask of triton_unified_attention.py:
// 577-590).  Optional attention sinks (s_aux, one logit per query head, in
// the units of scale * q . k) join the softmax's denominator only, once per
// row: out = sum_t e^(s_t - m) V_t / (sum_t e^(s_t - m) + e^(sink - m)), as
// init_softmax_M seeds M = sink, L = 1 (infra/triton_attention_helpers.py)
// and reduce_segments adds it once across segments.
// K/V rows of sequence b are gathered through block_tables[b, t / block_size]
// from NHD pages [num_blocks, block_size, Hk, D]; kv head = hq / (Hq/Hk).  This is
// FlashAttnDecode.forward (fastkernels/tasks/baseline/L1/flash_attn_decode.py:
// 113-181) and the reference's torch fallback Attention._decode_torch
// (fastkernels/tasks/baseline/L2/attention_impl.py:592-664).  Segments of a
// sequence are merged with the log-sum-exp rule of reduce_segments
// (triton_unified_attention.py:741-776): M = max m_s, L = sum l_s e^(m_s - M),
// O = sum o_s e^(m_s - M) / L, and O = 0 when L = 0.  fp8 KV pages are
// dequantised per kv head as float(x) * scale, the per-tensor rule of
// _cast_kv_tile (triton_unified_attention.py:51-67): k_scale is folded into the
// score scale and v_scale into the output, which is algebraically the same.
//
// Work decomposition.  A work-group has one wave64 per kv head (up to 8); the
// waves of a group stream the same token rows of the NHD cache, so each
// token's Hk * 256-byte row is read whole within a short window.  Two
// schedules share the per-wave tile loop:
//   balanced (default): the 16-token tiles of all sequences are concatenated
//     and cut into one equal range per work-group, with one work-group per
//     CU.  A sequence wholly inside a range is finished in place; a sequence
//     cut by range boundaries leaves one partial per range, merged by a
//     second kernel.  Every group streams the same number of bytes, so
//     sequences of 512 and 8192 tokens leave no idle tail.
//   fixed partitions (explicit num_splits): work-group = (partition p of
//     part_tokens tokens, sequence b), the classic flash-decoding split.
//
// MFMA mapping: fk_attn_tile.h, with the G query heads of a kv head as the
// 16 query columns of each tile.  Rows j >= G of the 16-row MFMA tiles are padding (zero Q, zero P): the matrix
// cores have ~80x the throughput this HBM-bound loop needs, so the padding is
// free, while the VALU work per token stays at a few instructions (no
// cross-lane dot-product reductions, two row-swap permutes per tile for the max).
#include "fk_attn_tile.h"

namespace fk {
namespace {

struct DecodeParams {
  uint16_t* out;
  int64_t out_row_stride;
  const uint16_t* q;
  int64_t q_row_stride;
  const uint8_t* k_cache;  // byte pointers; element size from the template
  const uint8_t* v_cache;
  const float* k_scale;
  const float* v_scale;
  const int32_t* block_tables;
  int64_t bt_row_stride;
  const int32_t* ctx_lens;
  int num_kv_heads;
  int gqa;
  int block_size_log2;
  int part_tokens;
  int max_parts;
  int64_t num_blocks;
  float scale_log2;  // softmax scale * log2(e)
  float* part_o;     // partial outputs (unnormalised), rows of 128 floats
  float* part_ml;    // per partial row: (max, sum) in the log2 domain
  int32_t* tile_off; // balanced schedule: [batch + 1] tile prefix sums, then range size
  int batch;
  int num_groups;    // balanced schedule: work-groups per kv-head group
  int window_left;   // sliding window: keys >= ctx - 1 - window_left (-1: none)
  const float* sinks;  // attention sink logits [num_heads] fp32, or nullptr
  // Fused store (fk_store_paged_decode); new_k == nullptr for a plain decode.
  // Row b of new_k / new_v (cache element type, heads contiguous) is sequence
  // b's new token, stored at slot slot_mapping[b] (skipped when out of range).
  const uint8_t* new_k;
  const uint8_t* new_v;
  int64_t new_k_stride;  // bytes between the rows of new_k
  int64_t new_v_stride;
  int slot_is_i64;
};

// Page id of token `tok` of sequence b, or -1 when the block-table entry is
// negative, >= num_blocks, or past the row (index >= bt_row_stride): such a
// page is masked and never read.  `bt` comes straight from a __restrict__
// kernel argument so that this wave-uniform read is a scalar load (lgkmcnt):
// a vector load here would make the compiler drain every outstanding KV load
// (vmcnt(0)) before the next tile's loads could issue.
__device__ __forceinline__ int64_t page_of(const DecodeParams& P, const int32_t* __restrict__ bt,
                                           int b, int tok) {
  const int idx = tok >> P.block_size_log2;
  if (idx >= P.bt_row_stride) return -1;
  const int64_t page = bt[b * P.bt_row_stride + idx];
  return (page >= 0 && page < P.num_blocks) ? page : -1;
}

// First visible key of a sequence of ctx tokens under the sliding window.
__device__ __forceinline__ int key_lo(const DecodeParams& P, int ctx) {
  return P.window_left >= 0 ? max(0, ctx - 1 - P.window_left) : 0;
}

// Sink logit of query head hq in the kernel's log2 units (scale * q . k
// scaled by log2(e)), or -inf without sinks.
__device__ __forceinline__ float sink_log2(const DecodeParams& P, int hq) {
  return P.sinks ? P.sinks[hq] * kLog2e : kNegInf;
}

// Issues the loads of one tile from page `page` (>= 0, < num_blocks).  Loads
// are unconditional so that every pipeline stage has the same number of loads
// in flight and the compiler can wait for one stage with vmcnt(N) instead of
// draining the queue; masked pages and tiles past the end load a safe page and
// are discarded by the consumer.  Fused store: tile row j (-1: none) is read
// from the new K/V row (nk / nv, this kv head's slice) instead of the cache,
// by selecting each lane's address, so the loop has no extra control flow.
template <bool kFp8>
__device__ __forceinline__ void load_tile(const DecodeParams& P, int64_t page, int h, int tok0,
                                          int r, int g, TileRegs<kFp8>& t, int j = -1,
                                          const uint8_t* nk = nullptr,
                                          const uint8_t* nv = nullptr) {
  const int bs_mask = (1 << P.block_size_log2) - 1;
  const int64_t slot0 = (page << P.block_size_log2) + (tok0 & bs_mask);
  constexpr int kElem = kFp8 ? 1 : 2;
  const int64_t row_bytes = static_cast<int64_t>(P.num_kv_heads) * kHead * kElem;
  const int64_t head_off = static_cast<int64_t>(h) * kHead * kElem;
  const uint8_t* krow = P.k_cache + (slot0 + r) * row_bytes + head_off;
  if (r == j) krow = nk;
  const uint8_t* vrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    vrow[i] = P.v_cache + (slot0 + 4 * g + i) * row_bytes + head_off;
    if (4 * g + i == j) vrow[i] = nv;
  }
  if constexpr (!kFp8) {
    // Per instruction: 16 rows x 64 contiguous bytes.
#pragma unroll
    for (int c = 0; c < 4; ++c)
      t.k[c] = ld16(krow + (32 * c + 8 * g) * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) t.v[i] = ld16(vrow[i] + 8 * r * 2);
  } else {
    t.k[0] = ld16(krow + 32 * g);
    t.k[1] = ld16(krow + 32 * g + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) t.v[i] = ld8(vrow[i] + 8 * r);
  }
}

// ---------------------------------------------------------------------------
// Fused store.  Sequence b's new token is at position p = ctx - 1.  The wave
// that streams p's tile (one per kv head) loads b's new K/V row up front and,
// when slot_mapping[b] is the slot of p in b's block table (the decode step),
// uses it in place of the cache row at p, then writes it to the cache after
// its tile loop, so no load waits for the store.  A slot that is not p's
// ("orphan") is written by that same wave, or, when no wave streams p (no
// context, or p past the launch's partitions), by a designated work-group; the
// order of an orphan write against other reads of its slot is unspecified.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t slot_of(const DecodeParams& P, const void* __restrict__ sm,
                                           int b) {
  return P.slot_is_i64 ? static_cast<const int64_t*>(sm)[b]
                       : static_cast<int64_t>(static_cast<const int32_t*>(sm)[b]);
}

// The raw 32-bit words of slot_mapping[b] (both halves of an int64 entry, or
// the int32 entry twice), loaded at computed indices without a branch so that
// they issue with the wave's first page lookups; slot_value() combines them
// behind a compiler barrier, so the wait for them lands where the slot is used.
struct SlotWords {
  int32_t lo, hi;
};
__device__ __forceinline__ SlotWords slot_words(const DecodeParams& P,
                                                const void* __restrict__ sm, int b) {
  const int32_t* s32 = static_cast<const int32_t*>(sm);
  const int w = P.slot_is_i64;  // 0 or 1
  const int i = b << w;
  return SlotWords{s32[i], s32[i + w]};
}
__device__ __forceinline__ int64_t slot_value(const DecodeParams& P, SlotWords s) {
  asm volatile("" : "+s"(s.lo), "+s"(s.hi));
  const int64_t wide = static_cast<int64_t>(
      (static_cast<uint64_t>(static_cast<uint32_t>(s.hi)) << 32) | static_cast<uint32_t>(s.lo));
  return P.slot_is_i64 ? wide : static_cast<int64_t>(s.lo);
}

// In-range slot of sequence b's new row, or -1.
__device__ __forceinline__ int64_t valid_slot(const DecodeParams& P, const void* __restrict__ sm,
                                              int b) {
  const int64_t slot = slot_of(P, sm, b);
  return (slot >= 0 && slot < (P.num_blocks << P.block_size_log2)) ? slot : -1;
}

// Writes kv head h of sequence b's new K and V rows to cache slot `slot`.
template <bool kFp8>
__device__ __forceinline__ void store_new_row(const DecodeParams& P, int b, int h, int64_t slot,
                                              int lane) {
  store_new_chunk<kFp8>(P, slot, h, lane, load_new_chunk<kFp8>(P, b, h, lane));
}

// One 16-byte chunk of sequence b's new K/V row for kv head h, in the layout
// store_new_chunk writes: lanes 0..15 hold K chunk (lane & 15), lanes 16..31 V
// chunk (lane & 15); chunk indices past the row (fp8) and lanes >= 32 re-read a
// valid chunk and are not stored.
template <bool kFp8>
__device__ __forceinline__ uint4 load_new_chunk(const DecodeParams& P, int b, int h, int lane) {
  constexpr int kElem = kFp8 ? 1 : 2;
  constexpr int kChunks = kHead * kElem / 16;
  const int c = min(lane & 15, kChunks - 1);
  const int64_t head_off = static_cast<int64_t>(h) * kHead * kElem;
  const bool is_v = (lane & 16) != 0;
  const uint8_t* src = (is_v ? P.new_v + b * P.new_v_stride : P.new_k + b * P.new_k_stride) +
                       head_off + 16 * c;
  return ld16(src);
}
template <bool kFp8>
__device__ __forceinline__ void store_new_chunk(const DecodeParams& P, int64_t slot, int h,
                                                int lane, const uint4& v) {
  constexpr int kElem = kFp8 ? 1 : 2;
  constexpr int kChunks = kHead * kElem / 16;
  const int c = lane & 15;
  if (lane >= 32 || c >= kChunks) return;
  const int64_t row_bytes = static_cast<int64_t>(P.num_kv_heads) * kHead * kElem;
  uint8_t* dst = const_cast<uint8_t*>((lane & 16) ? P.v_cache : P.k_cache) + slot * row_bytes +
                 static_cast<int64_t>(h) * kHead * kElem + 16 * c;
  *reinterpret_cast<uint4*>(dst) = v;
}

// Online-softmax state of one wave over the G query heads of one kv head, and
// the tile loop that streams a token range [tok_begin, tok_end) of a sequence
// through it (tok_begin a multiple of 16).
template <int kG, bool kFp8, int U, bool kStore>
struct WaveState {
  float m_run;  // running max of column r (same in the 4 lanes of a column)
  float l_run;  // this lane's share of the running sum of column r
  floatx4_t o[8];

  // kStore: when the segment ends at the context end (tok_end == ctx) and
  // slot_mapping[b] is the slot of position ctx - 1, that position's K/V are
  // read from sequence b's new row instead of the cache (load_tile's row j),
  // and the row (one 16-byte chunk per lane, loaded up front) is written to the
  // cache after the loop, so no load waits for the store.
  // Keys below key_lo (the sliding window's start) are masked; tok_begin is
  // the start of the tile holding key_lo or later.
  __device__ __forceinline__ void run(const DecodeParams& P, const int32_t* __restrict__ bt,
                                      const void* __restrict__ sm, int b, int h, int tok_begin,
                                      int tok_end, int ctx, int key_lo, int r, int g) {
    const int gqa = P.gqa;
    SlotWords sw{-1, -1};
    uint4 new_chunk = make_uint4(0, 0, 0, 0);  // this lane's chunk of b's new row
    const uint8_t* nk = nullptr;  // b's new K / V row, kv head h
    const uint8_t* nv = nullptr;
    int ftok0 = -1;  // first token of the tile holding ctx - 1, if this segment ends there
    if constexpr (kStore) {
      constexpr int kElem = kFp8 ? 1 : 2;
      const int64_t head_off = static_cast<int64_t>(h) * kHead * kElem;
      nk = P.new_k + b * P.new_k_stride + head_off;
      nv = P.new_v + b * P.new_v_stride + head_off;
      new_chunk = load_new_chunk<kFp8>(P, b, h, 16 * g + r);
      sw = slot_words(P, sm, b);
      if (tok_end == ctx && ctx > tok_begin)
        ftok0 = tok_begin + kTile * ((ctx - 1 - tok_begin) / kTile);
    }
    const bool head_ok = r < gqa;
    // Q^T operand: column r = query head h*G + r; dims permuted as the K loads.
    bf16x8_t qb[4];
    {
      const uint16_t* qp = P.q + b * P.q_row_stride + static_cast<int64_t>(h * gqa + r) * kHead;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d0 = kFp8 ? 32 * g + 8 * c : 32 * c + 8 * g;
        uint4 v = head_ok ? *reinterpret_cast<const uint4*>(qp + d0) : make_uint4(0, 0, 0, 0);
        qb[c] = __builtin_bit_cast(bf16x8_t, v);
      }
    }
    float s2 = P.scale_log2;
    if (kFp8 && P.k_scale) s2 *= P.k_scale[h];

    m_run = kNegInf;
    l_run = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) o[d] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    // Visible tokens are [key_lo, tok_end): one unsigned compare of tok - key_lo
    // against their count checks both bounds.
    const uint32_t span = static_cast<uint32_t>(tok_end - key_lo);
    // One 16-token tile: scores, online softmax update, P.V accumulation.
    auto process = [&](int tok0, int64_t page, const TileRegs<kFp8>& cur) {
      const int rel0 = tok0 + 4 * g - key_lo;
      uint4 kc[4];
      k_chunks(cur, kc);
      const floatx4_t acc = qk_scores(kc, qb);
      float s[4];
      float mt = kNegInf;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = head_ok && page >= 0 && static_cast<uint32_t>(rel0 + i) < span;
        s[i] = ok ? acc[i] * s2 : kNegInf;
        mt = fmaxf(mt, s[i]);
      }
      mt = pair_max(mt);  // max over the column's 4 lane groups (16 tokens)
      const float m_new = fmaxf(m_run, mt);
      const float m_use = m_new == kNegInf ? 0.f : m_new;
      // alpha = 1 for columns that have seen no valid score (their O and l are 0).
      const float alpha = m_new == kNegInf ? 1.f : __builtin_amdgcn_exp2f(m_run - m_use);
      float pr[4];
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[i] = __builtin_amdgcn_exp2f(s[i] - m_use);
        psum += pr[i];
      }
      l_run = l_run * alpha + psum;
      m_run = m_new;
      // Rescale O rows when some column max moved (rare after the first tiles).
      if (__ballot(alpha != 1.f) != 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = row_value<kG>(alpha, g, i);
#pragma unroll
          for (int d = 0; d < 8; ++d) o[d][i] *= a;
        }
      }
      const short4_t pa = p_operand(pr);
      // V rows past the context (inside a valid page) may hold anything: zero
      // them so that P = 0 never meets a NaN.
      uint4 vr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        vr[i] = (page >= 0 && static_cast<uint32_t>(rel0 + i) < span) ? v_row(cur, i)
                                                                     : make_uint4(0, 0, 0, 0);
      pv_accumulate(o, pa, vr);
    };

    const int ntiles = (tok_end - tok_begin + kTile - 1) / kTile;
    // The last block-table entry looked up (wave-uniform): a page holds
    // block_size / 16 tiles, so most tiles reuse it instead of a scalar load.
    int pc_idx = -1;
    int64_t pc_page = -1;
    // Issues the loads of tiles t0 .. t0+U-1 into `buf` (unconditional; tiles
    // past the end re-read the last tile, which hits in cache).
    // Issues the loads of tiles t0 .. t0+U-1 into `buf` (unconditional; tiles
    // past the end re-read the last tile, which hits in cache).
    auto fetch = [&](int t0, TileRegs<kFp8>(&buf)[U], int64_t(&pg)[U]) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int tok0 = tok_begin + kTile * min(t0 + u, ntiles - 1);
        const int idx = tok0 >> P.block_size_log2;
        if (idx != pc_idx) {
          pc_page = page_of(P, bt, b, tok0);
          pc_idx = idx;
        }
        pg[u] = pc_page;
        int j = -1;
        if constexpr (kStore) {
          // Fused when b's slot is that of position ctx - 1: in this tile's page
          // (a tile never spans pages), at offset (ctx - 1) mod block_size.
          // Branch-free (selects), so the load sequence stays one block.  (Peeling
          // the last chunk, the only one that can hold ctx - 1, out of the loop
          // measured no faster.)
          const int64_t want = (pg[u] << P.block_size_log2) +
                               ((ctx - 1) & ((1 << P.block_size_log2) - 1));
          const bool hit = tok0 == ftok0 && pg[u] >= 0 && slot_value(P, sw) == want;
          j = hit ? ctx - 1 - tok0 : -1;
        }
        load_tile<kFp8>(P, pg[u] < 0 ? 0 : pg[u], h, tok0, r, g, buf[u], j, nk, nv);
      }
    };
    auto consume = [&](int t0, const TileRegs<kFp8>(&buf)[U], const int64_t(&pg)[U]) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (t0 + u < ntiles) process(tok_begin + kTile * (t0 + u), pg[u], buf[u]);
      }
    };
    // Chunks of U tiles: issue all U tiles' loads, then consume them in order
    // (the compiler waits for tile u with vmcnt = loads issued after it).
    for (int t0 = 0; t0 < ntiles; t0 += U) {
      TileRegs<kFp8> buf[U];
      int64_t pg[U];
      fetch(t0, buf, pg);
      consume(t0, buf, pg);
    }
    // Column sums of l over the 4 lane groups: every lane of column j holds l_j.
    l_run = pair_sum(l_run);
    // The wave that streamed position ctx - 1 writes b's row: at that position
    // (fused) or, for any other in-range slot, there (an orphan).
    if (kStore && ftok0 >= 0) {
      const int64_t slot = slot_value(P, sw);
      if (slot >= 0 && slot < (P.num_blocks << P.block_size_log2))
        store_new_chunk<kFp8>(P, slot, h, 16 * g + r, new_chunk);
    }
  }

  // Normalised output row(s) of kv head h for a sequence finished in place.
  // Lane (r, g) holds O[head 4g+i][dims 8r .. 8r+7].
  __device__ __forceinline__ void write_final(const DecodeParams& P, int b, int h, int r,
                                              int g) const {
    const float vs = (kFp8 && P.v_scale) ? P.v_scale[h] : 1.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * g + i;
      float l = row_value<kG>(l_run, g, i);
      if (P.sinks) l = with_sink(l, row_value<kG>(m_run, g, i), sink_log2(P, h * P.gqa + (j < P.gqa ? j : 0)));
      if (j >= kG || j >= P.gqa) continue;
      const float f = l > 0.f ? vs / l : 0.f;
      uint32_t w[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const bf16x2_t pk = {static_cast<__bf16>(o[2 * d][i] * f),
                             static_cast<__bf16>(o[2 * d + 1][i] * f)};
        w[d] = __builtin_bit_cast(uint32_t, pk);
      }
      *reinterpret_cast<uint4*>(P.out + b * P.out_row_stride +
                                static_cast<int64_t>(h * P.gqa + j) * kHead + 8 * r) =
          make_uint4(w[0], w[1], w[2], w[3]);
    }
  }

  // Unnormalised partial (O scaled by v_scale, and (max, sum)) into partial
  // rows row0 + j, j < G.
  __device__ __forceinline__ void write_partial(const DecodeParams& P, int64_t row0, int h, int r,
                                                int g) const {
    const float vs = (kFp8 && P.v_scale) ? P.v_scale[h] : 1.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * g + i;
      if (j >= kG || j >= P.gqa) continue;
      float* dst = P.part_o + (row0 + j) * kHead + 8 * r;
      *reinterpret_cast<float4*>(dst) =
          make_float4(o[0][i] * vs, o[1][i] * vs, o[2][i] * vs, o[3][i] * vs);
      *reinterpret_cast<float4*>(dst + 4) =
          make_float4(o[4][i] * vs, o[5][i] * vs, o[6][i] * vs, o[7][i] * vs);
    }
    if (g == 0 && r < P.gqa) {
      P.part_ml[(row0 + r) * 2 + 0] = m_run;
      P.part_ml[(row0 + r) * 2 + 1] = l_run;
    }
  }
};

// Fixed partitions: work-group = (partition p, kv-head group, sequence b);
// wave w owns kv head h = blockIdx.y * NH + w and streams the partition.
// Partial rows: ((b * Hk + h) * max_parts + p) * G + j.
template <int NH, int kG, bool kFp8, int U, bool kStore>
__global__ __launch_bounds__(NH * 64) void paged_decode_partition_kernel(
    DecodeParams P, const int32_t* __restrict__ block_tables, const int32_t* __restrict__ ctx_lens,
    const void* __restrict__ slot_mapping) {
  const int p = blockIdx.x;
  const int b = blockIdx.z;
  const int ctx = ctx_lens[b];
  const int tok_begin = p * P.part_tokens;
  // Wave index made provably uniform so that page lookups are scalar loads.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = blockIdx.y * NH + wave;
  if (h >= P.num_kv_heads) return;  // uniform over the wave; no barriers follow
  const int lane = threadIdx.x & 63;
  if (tok_begin < ctx) {  // uniform over the work-group
    // The launch has max_parts partitions; the last one runs on to the context
    // end, so a context longer than the plan's max_seq_len bound (a graph
    // replayed after contexts grew) is still attended whole.
    const int tok_end = p == P.max_parts - 1 ? ctx : min(ctx, tok_begin + P.part_tokens);
    const int nparts = min((ctx + P.part_tokens - 1) / P.part_tokens, P.max_parts);
    const int r = lane & 15;
    const int g = lane >> 4;
    // Under a sliding window a partition starts no earlier than the tile of the
    // window's first key; one wholly before it streams nothing and leaves an
    // empty partial (max -inf, sum 0).
    const int lo = key_lo(P, ctx);
    WaveState<kG, kFp8, U, kStore> st;
    st.run(P, block_tables, slot_mapping, b, h, max(tok_begin, lo & ~(kTile - 1)), tok_end, ctx,
           lo, r, g);
    if (nparts == 1) {
      st.write_final(P, b, h, r, g);
    } else {
      const int64_t row0 =
          ((static_cast<int64_t>(b) * P.num_kv_heads + h) * P.max_parts + p) * P.gqa;
      st.write_partial(P, row0, h, r, g);
    }
  }
  // No partition streams position ctx - 1 (no context): partition 0 writes b's
  // row.
  if (kStore && p == 0 && ctx <= 0) {
    const int64_t os = valid_slot(P, slot_mapping, b);
    if (os >= 0) store_new_row<kFp8>(P, b, h, os, lane);
  }
}

// Tiles a sequence of ctx tokens streams: from the tile of its first visible
// key (the sliding window's start) to the end.
__device__ __forceinline__ int tiles_of(const DecodeParams& P, int ctx) {
  return ctx > 0 ? (ctx + kTile - 1) / kTile - key_lo(P, ctx) / kTile : 0;
}

// Balanced schedule: work-group w (of num_groups per kv-head group) takes
// tiles [w * S, (w+1) * S) of the concatenation of all sequences' tiles,
// S = ceil(total / num_groups).  Partial rows of a cut sequence:
// ((w * 2 + slot) * Hk + h) * G + j, slot 0 = the group's first segment,
// slot 1 = its last (a group holds at most one cut sequence at each end).
template <int NH, int kG, bool kFp8, int U, bool kStore>
__global__ __launch_bounds__(NH * 64) void paged_decode_balanced_kernel(
    DecodeParams P, const int32_t* __restrict__ block_tables, const int32_t* __restrict__ ctx_lens,
    const void* __restrict__ slot_mapping) {
  extern __shared__ int32_t toff[];  // [batch + 1] tile prefix sums
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int batch = P.batch;
  if (wave == 0) {
    int carry = 0;
    for (int base = 0; base < batch; base += 64) {
      const int i = base + lane;
      int v = i < batch ? tiles_of(P, ctx_lens[i]) : 0;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(v, off, 64);
        if (lane >= off) v += y;
      }
      if (i < batch) toff[i + 1] = carry + v;
      carry += __shfl(v, 63, 64);
    }
    if (lane == 0) toff[0] = 0;
  }
  __syncthreads();
  const int total = toff[batch];
  const int S = max(1, (total + P.num_groups - 1) / P.num_groups);
  const int w = blockIdx.x;
  if (w == 0 && blockIdx.y == 0) {  // publish the schedule for the merge kernel
    for (int i = threadIdx.x; i <= batch; i += blockDim.x) P.tile_off[i] = toff[i];
    if (threadIdx.x == 0) P.tile_off[batch + 1] = S;
  }
  const int h = blockIdx.y * NH + wave;
  if (h >= P.num_kv_heads) return;  // uniform over the wave; no barriers follow
  const int t_lo = w * S;
  const int t_hi = min(total, t_lo + S);
  if (t_lo < total) {
    const int r = lane & 15;
    const int g = lane >> 4;
    // First sequence with tiles at t_lo: largest b with toff[b] <= t_lo.
    int lo = 0, hi = batch;  // invariant: toff[lo] <= t_lo < toff[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (toff[mid] <= t_lo) lo = mid; else hi = mid;
    }
    WaveState<kG, kFp8, U, kStore> st;
    for (int b = lo; b < batch && toff[b] < t_hi; ++b) {
      const int s_lo = max(t_lo, toff[b]) - toff[b];
      const int s_hi = min(t_hi, toff[b + 1]) - toff[b];
      if (s_hi <= s_lo) continue;  // empty sequence
      const int ctx = ctx_lens[b];
      const int lo = key_lo(P, ctx);
      const int t_first = lo / kTile;  // the sequence's tile s is its tile t_first + s
      st.run(P, block_tables, slot_mapping, b, h, kTile * (t_first + s_lo),
             min(ctx, kTile * (t_first + s_hi)), ctx, lo, r, g);
      if (toff[b] >= t_lo && toff[b + 1] <= t_hi) {
        st.write_final(P, b, h, r, g);
      } else {
        const int slot = toff[b] <= t_lo ? 0 : 1;
        const int64_t row0 = ((static_cast<int64_t>(w) * 2 + slot) * P.num_kv_heads + h) * P.gqa;
        st.write_partial(P, row0, h, r, g);
      }
    }
  }
  // Sequences without tiles (no context) have no wave that streams their
  // last position: group w writes the rows of those with b = w mod G.
  if (kStore) {
    for (int b = w; b < batch; b += P.num_groups) {
      if (toff[b + 1] != toff[b]) continue;
      const int64_t os = valid_slot(P, slot_mapping, b);
      if (os >= 0) store_new_row<kFp8>(P, b, h, os, lane);
    }
  }
}

// Merge of one (query head hq, sequence b) by one wave; each lane owns two
// dims.  Partial rows: k = 0 is `alt_first_row`, k >= 1 is first_row + k *
// row_stride.  The pieces are taken kMergeBatch at a time (one batch for up to
// 64 pieces): lane k loads piece k's (max, sum) while the wave issues the O
// loads of every piece in the batch, all independent, so the merge costs one
// load latency; the batch max and sum are wave reductions, and a running
// (M, L, O) carries across batches with the reduce_segments rescaling.
constexpr int kMergeBatch = 64;  // pieces per batch: one (max, sum) per lane
constexpr int kMergeUnroll = 8;  // O rows in flight per wave
constexpr int kMergeWaves = 4;   // independent merge rows per work-group
__device__ __forceinline__ void merge_rows(uint16_t* orow, const float* part_o,
                                           const float* part_ml, int64_t first_row,
                                           int64_t row_stride, int nrows, int64_t alt_first_row,
                                           float sink2, int lane) {
  auto row_of = [&](int k) -> int64_t { return k == 0 ? alt_first_row : first_row + k * row_stride; };
  float M = kNegInf, L = 0.f, o0 = 0.f, o1 = 0.f;
  for (int k0 = 0; k0 < nrows; k0 += kMergeBatch) {
    const int n = min(kMergeBatch, nrows - k0);
    // (max, sum) of piece k0 + lane; lanes past the batch hold an empty piece.
    float m = kNegInf, l = 0.f;
    if (lane < n) {
      const float2 ml = *reinterpret_cast<const float2*>(part_ml + row_of(k0 + lane) * 2);
      m = ml.x;
      l = ml.y;
    }
    // O of the batch's pieces, kMergeUnroll rows in flight at a time.
    float2 ov[kMergeUnroll];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u)
      ov[u] = u < n ? reinterpret_cast<const float2*>(part_o + row_of(k0 + u) * kHead)[lane]
                    : make_float2(0.f, 0.f);
    const float mb = wave_max(m);
    const float mn = fmaxf(M, mb);
    if (mn == kNegInf) continue;  // no valid piece yet (all rows empty)
    const float a = __builtin_amdgcn_exp2f(M - mn);  // 0 when M = -inf
    const float f = __builtin_amdgcn_exp2f(m - mn);  // lane k's weight; 0 for empty pieces
    L = L * a + wave_sum(l * f);
    o0 *= a;
    o1 *= a;
    for (int u0 = 0; u0 < n; u0 += kMergeUnroll) {
      if (u0 > 0) {
#pragma unroll
        for (int u = 0; u < kMergeUnroll; ++u)
          ov[u] = u0 + u < n
                      ? reinterpret_cast<const float2*>(part_o + row_of(k0 + u0 + u) * kHead)[lane]
                      : make_float2(0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < kMergeUnroll; ++u) {
        const float w = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), min(u0 + u, 63)));
        if (u0 + u < n) {
          o0 = __builtin_fmaf(ov[u].x, w, o0);
          o1 = __builtin_fmaf(ov[u].y, w, o1);
        }
      }
    }
    M = mn;
  }
  L = with_sink(L, M, sink2);  // the sink joins the merged row once
  const float inv = L > 0.f ? 1.f / L : 0.f;
  const bf16x2_t pk = {static_cast<__bf16>(o0 * inv), static_cast<__bf16>(o1 * inv)};
  reinterpret_cast<uint32_t*>(orow)[lane] = __builtin_bit_cast(uint32_t, pk);
}

// Fixed partitions: merge sequences with more than one partition; zero empty ones.
// Work-group = kMergeWaves independent waves, wave v = query head
// blockIdx.x * kMergeWaves + v of sequence blockIdx.y.
__global__ __launch_bounds__(kMergeWaves * 64) void paged_decode_partition_reduce_kernel(
    DecodeParams P, int num_heads) {
  const int hq = blockIdx.x * kMergeWaves + (threadIdx.x >> 6);
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  if (hq >= num_heads) return;  // no barriers in this kernel
  const int ctx = P.ctx_lens[b];
  uint16_t* orow = P.out + b * P.out_row_stride + static_cast<int64_t>(hq) * kHead;
  if (ctx <= 0) {
    reinterpret_cast<uint32_t*>(orow)[lane] = 0u;
    return;
  }
  const int nparts = min((ctx + P.part_tokens - 1) / P.part_tokens, P.max_parts);
  if (nparts <= 1) return;  // written by the partition kernel
  const int h = hq / P.gqa;
  const int j = hq - h * P.gqa;
  const int64_t first = (static_cast<int64_t>(b) * P.num_kv_heads + h) * P.max_parts * P.gqa + j;
  merge_rows(orow, P.part_o, P.part_ml, first, P.gqa, nparts, first, sink_log2(P, hq), lane);
}

// Balanced schedule: merge sequences cut across work-groups; zero empty ones.
// Work-group = kMergeWaves independent waves, as the partition reduce.
__global__ __launch_bounds__(kMergeWaves * 64) void paged_decode_balanced_reduce_kernel(
    DecodeParams P, int num_heads) {
  const int hq = blockIdx.x * kMergeWaves + (threadIdx.x >> 6);
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  if (hq >= num_heads) return;  // no barriers in this kernel
  uint16_t* orow = P.out + b * P.out_row_stride + static_cast<int64_t>(hq) * kHead;
  const int t0 = P.tile_off[b];
  const int t1 = P.tile_off[b + 1];
  const int S = P.tile_off[P.batch + 1];
  if (t1 <= t0) {
    reinterpret_cast<uint32_t*>(orow)[lane] = 0u;
    return;
  }
  const int w0 = t0 / S;
  const int w1 = (t1 - 1) / S;
  if (w0 == w1) return;  // finished in place by work-group w0
  const int h = hq / P.gqa;
  const int j = hq - h * P.gqa;
  const int64_t hk = P.num_kv_heads;
  // Group w0 holds the sequence in slot 1 unless the sequence starts its range;
  // groups w0+1 .. w1 hold it in slot 0.
  const int slot0 = t0 > w0 * S ? 1 : 0;
  const int64_t first_alt = ((static_cast<int64_t>(w0) * 2 + slot0) * hk + h) * P.gqa + j;
  const int64_t first = ((static_cast<int64_t>(w0) * 2 + 0) * hk + h) * P.gqa + j;
  merge_rows(orow, P.part_o, P.part_ml, first, 2 * hk * P.gqa, w1 - w0 + 1, first_alt,
             sink_log2(P, hq), lane);
}

// Tuning knob (compile-time): tiles per load set.
#ifndef FK_DECODE_CHUNK
#define FK_DECODE_CHUNK 2
#endif
constexpr int kChunk = FK_DECODE_CHUNK;  // tiles loaded per wave per set
constexpr int kMaxWavesPerGroup = 8;     // kv heads (waves) per work-group
constexpr int kPartQuant = 64;           // fixed-partition granularity in tokens
constexpr int kMaxBalancedBatch = 8192;  // tile prefix sums live in LDS

int num_cus() {
  static int cached = -1;
  if (cached < 0) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess &&
        prop.multiProcessorCount > 0)
      cached = prop.multiProcessorCount;
    else
      cached = 256;  // MI355X
    (void)hipGetLastError();
  }
  return cached;
}

int waves_per_group(int num_kv_heads) {
  return num_kv_heads < kMaxWavesPerGroup ? num_kv_heads : kMaxWavesPerGroup;
}

// Workspace layout: part_o rows, part_ml rows (256-byte aligned), then (balanced
// only) batch + 2 int32 for the tile prefix sums and the range size.
int64_t o_region(int64_t rows) { return (rows * kHead * 4 + 255) / 256 * 256; }
int64_t ml_region(int64_t rows) { return (rows * 2 * 4 + 255) / 256 * 256; }

int64_t partial_rows(bool balanced, int64_t batch, int num_heads, int64_t max_parts) {
  // balanced: max_parts = work-groups per kv-head group, 2 slots each.
  return balanced ? max_parts * 2 * num_heads : batch * num_heads * max_parts;
}

int64_t workspace_bytes(bool balanced, int64_t batch, int num_heads, int64_t max_parts) {
  const int64_t rows = partial_rows(balanced, batch, num_heads, max_parts);
  return o_region(rows) + ml_region(rows) + (balanced ? (batch + 2) * 4 : 0);
}

int validate(const char* name, int64_t batch, int num_heads, int num_kv_heads, int head_size,
             int64_t part_tokens, int64_t max_parts) {
  FK_REQUIRE(batch >= 0 && batch <= 65535, "%s: batch %lld out of range [0, 65535]", name,
             (long long)batch);
  FK_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             "%s: num_heads %d must be a positive multiple of num_kv_heads %d", name, num_heads,
             num_kv_heads);
  if (head_size != kHead)
    return set_error(FK_ERR_UNSUPPORTED, "%s: head_size %d unsupported (128 only)", name,
                     head_size);
  if (num_heads / num_kv_heads > 16)
    return set_error(FK_ERR_UNSUPPORTED, "%s: GQA group %d > 16 unsupported", name,
                     num_heads / num_kv_heads);
  if (part_tokens == 0) {
    FK_REQUIRE(batch <= kMaxBalancedBatch, "%s: balanced schedule supports batch <= %d", name,
               kMaxBalancedBatch);
  } else {
    FK_REQUIRE(part_tokens > 0 && part_tokens % kPartQuant == 0 && part_tokens <= (1 << 30),
               "%s: part_tokens %lld must be 0 (balanced) or a positive multiple of %d", name,
               (long long)part_tokens, kPartQuant);
  }
  FK_REQUIRE(max_parts > 0 && max_parts <= 65535, "%s: max_parts %lld out of range", name,
             (long long)max_parts);
  return FK_OK;
}

struct Launch {
  DecodeParams P;
  const void* slot_mapping = nullptr;
  bool balanced;
  bool fp8;
  int nh;
  dim3 grid;
};

int prepare(const char* name, Launch& L, void* out, int64_t out_row_stride, const void* q,
            int64_t q_row_stride, const void* k_cache, const void* v_cache, int kv_dtype,
            const float* k_scale, const float* v_scale, const int32_t* block_tables,
            int64_t bt_row_stride, const int32_t* ctx_lens, int64_t batch, int num_heads,
            int num_kv_heads, int head_size, int block_size, int64_t num_blocks, float scale,
            int window_left, const float* sinks, int64_t part_tokens, int64_t max_parts,
            void* workspace, int64_t ws_bytes) {
  int rc = validate(name, batch, num_heads, num_kv_heads, head_size, part_tokens, max_parts);
  if (rc != FK_OK) return rc;
  FK_REQUIRE(window_left >= -1, "%s: window_left %d must be -1 (no window) or >= 0", name,
             window_left);
  FK_REQUIRE(block_size >= kTile && (block_size & (block_size - 1)) == 0,
             "%s: block_size %d must be a power of two >= 16", name, block_size);
  FK_REQUIRE(kv_dtype == FK_DTYPE_BF16 || kv_dtype == FK_DTYPE_FP8_E4M3FN,
             "%s: kv dtype %d unsupported (bf16 or fp8 e4m3fn)", name, kv_dtype);
  FK_REQUIRE(q_row_stride >= static_cast<int64_t>(num_heads) * head_size &&
                 out_row_stride >= static_cast<int64_t>(num_heads) * head_size,
             "%s: row stride shorter than num_heads * head_size", name);
  if (batch == 0) return FK_OK;
  FK_REQUIRE(out && q && k_cache && v_cache && block_tables && ctx_lens, "%s: null pointer",
             name);
  FK_REQUIRE(num_blocks >= 1, "%s: the cache must hold at least one block", name);
  FK_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out) &&
                 q_row_stride % 8 == 0 && out_row_stride % 8 == 0,
             "%s: q/out/cache must be 16-byte aligned with rows a multiple of 8 elements", name);
  const bool balanced = part_tokens == 0;
  const bool needs_ws = balanced || max_parts > 1;
  const int64_t need = workspace_bytes(balanced, batch, num_heads, max_parts);
  if (needs_ws && (workspace == nullptr || ws_bytes < need))
    return set_error(FK_ERR_WORKSPACE, "%s: workspace of %lld bytes < %lld required", name,
                     (long long)ws_bytes, (long long)need);
  FK_REQUIRE(!needs_ws || aligned16(workspace), "%s: workspace must be 16-byte aligned", name);

  DecodeParams& P = L.P;
  P.out = static_cast<uint16_t*>(out);
  P.out_row_stride = out_row_stride;
  P.q = static_cast<const uint16_t*>(q);
  P.q_row_stride = q_row_stride;
  P.k_cache = static_cast<const uint8_t*>(k_cache);
  P.v_cache = static_cast<const uint8_t*>(v_cache);
  P.k_scale = k_scale;
  P.v_scale = v_scale;
  P.block_tables = block_tables;
  P.bt_row_stride = bt_row_stride;
  P.ctx_lens = ctx_lens;
  P.num_kv_heads = num_kv_heads;
  P.gqa = num_heads / num_kv_heads;
  P.block_size_log2 = __builtin_ctz(static_cast<unsigned>(block_size));
  P.part_tokens = static_cast<int>(part_tokens);
  P.max_parts = static_cast<int>(max_parts);
  P.num_blocks = num_blocks;
  P.scale_log2 = scale * kLog2e;
  P.batch = static_cast<int>(batch);
  P.num_groups = static_cast<int>(max_parts);
  P.window_left = window_left;
  P.sinks = sinks;
  P.new_k = nullptr;
  P.new_v = nullptr;
  P.new_k_stride = P.new_v_stride = 0;
  P.slot_is_i64 = 0;
  const int64_t rows = partial_rows(balanced, batch, num_heads, max_parts);
  char* ws = static_cast<char*>(workspace);
  P.part_o = needs_ws ? reinterpret_cast<float*>(ws) : nullptr;
  P.part_ml = needs_ws ? reinterpret_cast<float*>(ws + o_region(rows)) : nullptr;
  P.tile_off = balanced ? reinterpret_cast<int32_t*>(ws + o_region(rows) + ml_region(rows))
                        : nullptr;
  L.balanced = balanced;
  L.fp8 = kv_dtype == FK_DTYPE_FP8_E4M3FN;
  L.nh = waves_per_group(num_kv_heads);
  const unsigned hgroups = static_cast<unsigned>((num_kv_heads + L.nh - 1) / L.nh);
  L.grid = balanced ? dim3(static_cast<unsigned>(max_parts), hgroups, 1)
                    : dim3(static_cast<unsigned>(max_parts), hgroups, static_cast<unsigned>(batch));
  return FK_OK;
}

template <int NH, int G, bool FP8, bool ST>
void launch_main_st(const Launch& L, hipStream_t stream) {
  if (L.balanced) {
    const size_t lds = static_cast<size_t>(L.P.batch + 1) * sizeof(int32_t);
    hipLaunchKernelGGL((paged_decode_balanced_kernel<NH, G, FP8, kChunk, ST>), L.grid,
                       dim3(NH * 64), lds, stream, L.P, L.P.block_tables, L.P.ctx_lens,
                       L.slot_mapping);
  } else {
    hipLaunchKernelGGL((paged_decode_partition_kernel<NH, G, FP8, kChunk, ST>), L.grid,
                       dim3(NH * 64), 0, stream, L.P, L.P.block_tables, L.P.ctx_lens,
                       L.slot_mapping);
  }
}

template <int NH, int G, bool FP8>
void launch_main(const Launch& L, hipStream_t stream) {
  if (L.P.new_k != nullptr)
    launch_main_st<NH, G, FP8, true>(L, stream);
  else
    launch_main_st<NH, G, FP8, false>(L, stream);
}

template <int G, bool FP8>
void launch_main_nh(const Launch& L, hipStream_t stream) {
  switch (L.nh) {
    case 1: launch_main<1, G, FP8>(L, stream); break;
    case 2: launch_main<2, G, FP8>(L, stream); break;
    case 4: launch_main<4, G, FP8>(L, stream); break;
    default: launch_main<8, G, FP8>(L, stream); break;
  }
}

template <int G>
void launch_main_g(const Launch& L, hipStream_t stream) {
  if (L.fp8)
    launch_main_nh<G, true>(L, stream);
  else
    launch_main_nh<G, false>(L, stream);
}

}  // namespace
}  // namespace fk

using namespace fk;

extern "C" int fk_paged_decode_plan(int64_t batch, int num_heads, int num_kv_heads, int head_size,
                                    int64_t max_seq_len, int num_splits, int64_t* part_tokens,
                                    int64_t* max_parts, int64_t* workspace_bytes_out) {
  FK_REQUIRE(part_tokens && max_parts && workspace_bytes_out,
             "fk_paged_decode_plan: null output pointer");
  FK_REQUIRE(batch >= 0 && num_heads > 0 && num_kv_heads > 0 && max_seq_len >= 0 &&
                 num_splits >= 0,
             "fk_paged_decode_plan: negative argument");
  const int64_t L = max_seq_len > 0 ? max_seq_len : 1;
  if (num_splits == 0 && batch <= kMaxBalancedBatch) {
    // Balanced: one work-group per CU for each kv-head group when a group
    // fills a CU (8 waves), proportionally more for fewer kv heads.
    const int nh = waves_per_group(num_kv_heads);
    *part_tokens = 0;
    *max_parts = static_cast<int64_t>(num_cus()) * (kMaxWavesPerGroup / nh);
  } else {
    int64_t part;
    if (num_splits > 0) {
      part = (L + num_splits - 1) / num_splits;
    } else {
      // ~8192 waves (one per (sequence, kv head, partition)), >= 256 tokens each.
      const int64_t units = (batch > 0 ? batch : 1) * num_kv_heads;
      part = (L * units + 8191) / 8192;
      if (part < 256) part = 256;
    }
    part = (part + kPartQuant - 1) / kPartQuant * kPartQuant;
    *part_tokens = part;
    *max_parts = (L + part - 1) / part;
  }
  (void)head_size;
  *workspace_bytes_out =
      batch > 0 ? workspace_bytes(*part_tokens == 0, batch, num_heads, *max_parts) : 0;
  return FK_OK;
}

extern "C" int fk_paged_decode_partials(
    void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride, const void* k_cache,
    const void* v_cache, int kv_dtype, const float* k_scale, const float* v_scale,
    const int32_t* block_tables, int64_t bt_row_stride, const int32_t* ctx_lens, int64_t batch,
    int num_heads, int num_kv_heads, int head_size, int block_size, int64_t num_blocks,
    float scale, int window_left, const float* sinks, int64_t part_tokens, int64_t max_parts,
    void* workspace, int64_t ws_bytes, void* stream) {
  Launch L;
  int rc = prepare("fk_paged_decode_partials", L, out, out_row_stride, q, q_row_stride, k_cache,
                   v_cache, kv_dtype, k_scale, v_scale, block_tables, bt_row_stride, ctx_lens,
                   batch, num_heads, num_kv_heads, head_size, block_size, num_blocks, scale,
                   window_left, sinks, part_tokens, max_parts, workspace, ws_bytes);
  if (rc != FK_OK || batch == 0) return rc;
  hipStream_t s = as_stream(stream);
  if (L.P.gqa <= 4)
    launch_main_g<4>(L, s);
  else if (L.P.gqa <= 8)
    launch_main_g<8>(L, s);
  else
    launch_main_g<16>(L, s);
  return check_launch("fk_paged_decode_partials");
}

extern "C" int fk_paged_decode_reduce(
    void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride, const void* k_cache,
    const void* v_cache, int kv_dtype, const float* k_scale, const float* v_scale,
    const int32_t* block_tables, int64_t bt_row_stride, const int32_t* ctx_lens, int64_t batch,
    int num_heads, int num_kv_heads, int head_size, int block_size, int64_t num_blocks,
    float scale, int window_left, const float* sinks, int64_t part_tokens, int64_t max_parts,
    void* workspace, int64_t ws_bytes, void* stream) {
  Launch L;
  int rc = prepare("fk_paged_decode_reduce", L, out, out_row_stride, q, q_row_stride, k_cache,
                   v_cache, kv_dtype, k_scale, v_scale, block_tables, bt_row_stride, ctx_lens,
                   batch, num_heads, num_kv_heads, head_size, block_size, num_blocks, scale,
                   window_left, sinks, part_tokens, max_parts, workspace, ws_bytes);
  if (rc != FK_OK || batch == 0) return rc;
  const dim3 grid(static_cast<unsigned>((num_heads + kMergeWaves - 1) / kMergeWaves),
                  static_cast<unsigned>(batch));
  if (L.balanced)
    hipLaunchKernelGGL(paged_decode_balanced_reduce_kernel, grid, dim3(kMergeWaves * 64), 0,
                       as_stream(stream), L.P, num_heads);
  else
    hipLaunchKernelGGL(paged_decode_partition_reduce_kernel, grid, dim3(kMergeWaves * 64), 0,
                       as_stream(stream), L.P, num_heads);
  return check_launch("fk_paged_decode_reduce");
}

extern "C" int fk_paged_decode(void* out, int64_t out_row_stride, const void* q,
                               int64_t q_row_stride, const void* k_cache, const void* v_cache,
                               int kv_dtype, const float* k_scale, const float* v_scale,
                               const int32_t* block_tables, int64_t bt_row_stride,
                               const int32_t* ctx_lens, int64_t batch, int num_heads,
                               int num_kv_heads, int head_size, int block_size,
                               int64_t num_blocks, float scale, int window_left,
                               const float* sinks, int64_t part_tokens, int64_t max_parts,
                               void* workspace, int64_t ws_bytes, void* stream) {
  int rc = fk_paged_decode_partials(out, out_row_stride, q, q_row_stride, k_cache, v_cache,
                                    kv_dtype, k_scale, v_scale, block_tables, bt_row_stride,
                                    ctx_lens, batch, num_heads, num_kv_heads, head_size,
                                    block_size, num_blocks, scale, window_left, sinks,
                                    part_tokens, max_parts, workspace, ws_bytes, stream);
  if (rc != FK_OK) return rc;
  return fk_paged_decode_reduce(out, out_row_stride, q, q_row_stride, k_cache, v_cache, kv_dtype,
                                k_scale, v_scale, block_tables, bt_row_stride, ctx_lens, batch,
                                num_heads, num_kv_heads, head_size, block_size, num_blocks, scale,
                                window_left, sinks, part_tokens, max_parts, workspace, ws_bytes,
                                stream);
}

extern "C" int fk_store_paged_decode(
    void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride, const void* key,
    int64_t key_row_stride, const void* value, int64_t value_row_stride, const void* slot_mapping,
    int slot_is_i64, void* k_cache, void* v_cache, int kv_dtype, const float* k_scale,
    const float* v_scale, const int32_t* block_tables, int64_t bt_row_stride,
    const int32_t* ctx_lens, int64_t batch, int num_heads, int num_kv_heads, int head_size,
    int block_size, int64_t num_blocks, float scale, int window_left, const float* sinks,
    int64_t part_tokens, int64_t max_parts, void* workspace, int64_t ws_bytes, void* stream) {
  const char* name = "fk_store_paged_decode";
  Launch L;
  int rc = prepare(name, L, out, out_row_stride, q, q_row_stride, k_cache, v_cache, kv_dtype,
                   k_scale, v_scale, block_tables, bt_row_stride, ctx_lens, batch, num_heads,
                   num_kv_heads, head_size, block_size, num_blocks, scale, window_left, sinks,
                   part_tokens, max_parts, workspace, ws_bytes);
  if (rc != FK_OK) return rc;
  const int64_t elem = kv_dtype == FK_DTYPE_FP8_E4M3FN ? 1 : 2;
  const int64_t row = static_cast<int64_t>(num_kv_heads) * kHead;
  FK_REQUIRE(key_row_stride >= row && value_row_stride >= row,
             "%s: key/value row stride shorter than num_kv_heads * head_size", name);
  if (batch == 0) return FK_OK;
  FK_REQUIRE(key && value && slot_mapping, "%s: null pointer", name);
  FK_REQUIRE(aligned16(key) && aligned16(value) && (key_row_stride * elem) % 16 == 0 &&
                 (value_row_stride * elem) % 16 == 0,
             "%s: key/value must be 16-byte aligned with 16-byte row strides", name);
  FK_REQUIRE(num_blocks <= (int64_t(1) << 40) / block_size, "%s: cache too large", name);
  L.P.new_k = static_cast<const uint8_t*>(key);
  L.P.new_v = static_cast<const uint8_t*>(value);
  L.P.new_k_stride = key_row_stride * elem;
  L.P.new_v_stride = value_row_stride * elem;
  L.P.slot_is_i64 = slot_is_i64 ? 1 : 0;
  L.slot_mapping = slot_mapping;
  hipStream_t s = as_stream(stream);
  if (L.P.gqa <= 4)
    launch_main_g<4>(L, s);
  else if (L.P.gqa <= 8)
    launch_main_g<8>(L, s);
  else
    launch_main_g<16>(L, s);
  rc = check_launch(name);
  if (rc != FK_OK) return rc;
  return fk_paged_decode_reduce(out, out_row_stride, q, q_row_stride, k_cache, v_cache, kv_dtype,
                                k_scale, v_scale, block_tables, bt_row_stride, ctx_lens, batch,
                                num_heads, num_kv_heads, head_size, block_size, num_blocks, scale,
                                window_left, sinks, part_tokens, max_parts, workspace, ws_bytes,
                                stream);
}
