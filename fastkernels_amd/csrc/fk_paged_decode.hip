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
// _cast_kv_tile (triton_unified_attention.py:51-67): each K and V element is
// float(x) * scale rounded to bf16 before it enters the MFMAs, as the reference
// casts the scaled tile to the query dtype.
// Head sizes D = 64, 128 and 256 (the reference builds FlashAttnDecode at 128,
// and at 256 and 64 for Qwen3-Next and Whisper, L2/qwen3_next_attention.py:
// 148-150, L2/whisper_attention.py:185-190) are template instantiations.
//
// Work decomposition.  A wave owns one "virtual head": a kv head and a block
// of up to 16 of its G query heads (the 16 query columns of an MFMA tile), so
// groups larger than 16 take ceil(G / 16) waves per kv head, which stream the
// same K/V rows.  A work-group has up to 8 such waves; the waves of a group
// stream the same token rows of the NHD cache, so each token's Hk * D-element
// row is read whole within a short window.  Two schedules share the per-wave
// tile loop:
//   balanced (default): the 16-token tiles of all sequences are concatenated
//     and cut into one equal range per work-group, with one work-group per
//     CU.  A sequence wholly inside a range is finished in place; a sequence
//     cut by range boundaries leaves one partial per range, merged by a
//     second kernel.  Every group streams the same number of bytes, so
//     sequences of 512 and 8192 tokens leave no idle tail.
//   fixed partitions (explicit num_splits): work-group = (partition p of
//     part_tokens tokens, sequence b), the classic flash-decoding split.
//
// MFMA mapping: fk_attn_tile.h.  Rows j >= G of the 16-row MFMA tiles are
// padding (zero Q, zero P): the matrix cores have ~80x the throughput this
// HBM-bound loop needs, so the padding is free, while the VALU work per token
// stays at a few instructions (no cross-lane dot-product reductions, two
// row-swap permutes per tile for the max).
//
// Two alternative tile forms are compiled in only for A/B measurement; the
// shipped library defines neither macro, and both measured slower on C3:
//   FK_DECODE_VALU_TILE  bf16, head size 128, groups of up to 4 query heads:
//     Q K^T and P V on the VALU (v_dot2_f32_bf16) instead of the matrix cores.
//   FK_DECODE_LDS_STAGE  bf16, head size 128, plain decode: K/V tiles go from
//     HBM straight to LDS (global_load_lds_dwordx4) through a two-stage ring
//     per wave, so the next tile's loads are in flight while a tile is used.
#include "fk_attn_tile.h"

namespace fk {
namespace {

// Lock step: the waves of a work-group stream the same token rows (one kv head
// each), and meet at a barrier every so many load sets, so that a row's
// kv-head slices are read together rather than drifting apart (the younger
// wave on each SIMD falls behind by several µs otherwise).  0 disables it; fp8
// pages (half the bytes per row) measured no gain from it.
#ifndef FK_DECODE_SYNC_CHUNKS
#define FK_DECODE_SYNC_CHUNKS 2
#endif
#ifndef FK_DECODE_SYNC_CHUNKS_FP8
#define FK_DECODE_SYNC_CHUNKS_FP8 0
#endif

#ifdef FK_DECODE_VALU_TILE
constexpr bool kValuBuild = true;
#else
constexpr bool kValuBuild = false;
#endif
#ifdef FK_DECODE_LDS_STAGE
constexpr bool kLdsBuild = true;
#else
constexpr bool kLdsBuild = false;
#endif

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
  int num_heads;
  int num_kv_heads;
  int gqa;           // query heads per kv head
  int col_blocks;    // waves per kv head: ceil(gqa / 16)
  int block_size_log2;
  int part_tokens;
  int max_parts;
  int64_t num_blocks;
  float scale_log2;  // softmax scale * log2(e)
  float* part_o;     // partial outputs (unnormalised), rows of D floats
  float* part_ml;    // per partial row: (max, sum) in the log2 domain
  int32_t* tile_off; // balanced schedule: [batch + 1] tile prefix sums, then range size
  int batch;
  int num_groups;    // balanced schedule: work-groups per virtual-head group
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
  // Fixed partitions: waves per virtual head (1 or 2).  With 2, each takes half
  // of the partition's tiles and the second leaves its state in LDS for the
  // first to merge (launches that would otherwise leave one wave per SIMD).
  int split;
};

// The query heads one wave handles: kv head kvh, query heads qbase .. qbase +
// ncols - 1 (a block of at most 16 of the kv head's group).
struct VHead {
  int kvh;
  int qbase;
  int ncols;
  bool first;  // the kv head's first column block (it writes the fused-store row)
};
__device__ __forceinline__ VHead vhead(const DecodeParams& P, int v) {
  VHead vh;
  vh.kvh = v / P.col_blocks;
  const int cb = v - vh.kvh * P.col_blocks;
  vh.qbase = vh.kvh * P.gqa + 16 * cb;
  vh.ncols = min(16, P.gqa - 16 * cb);
  vh.first = cb == 0;
  return vh;
}

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
// are discarded by the consumer.
template <bool kFp8, int D>
__device__ __forceinline__ void load_tile(const DecodeParams& P, int64_t page, int kvh, int tok0,
                                          int r, int g, DTile<kFp8, D>& t) {
  const int bs_mask = (1 << P.block_size_log2) - 1;
  const int64_t slot0 = (page << P.block_size_log2) + (tok0 & bs_mask);
  constexpr int kElem = kFp8 ? 1 : 2;
  const int64_t row_bytes = static_cast<int64_t>(P.num_kv_heads) * D * kElem;
  const int64_t head_off = static_cast<int64_t>(kvh) * D * kElem;
  const uint8_t* krow = P.k_cache + (slot0 + r) * row_bytes + head_off;
  const uint8_t* vrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) vrow[i] = P.v_cache + (slot0 + 4 * g + i) * row_bytes + head_off;
  if constexpr (!kFp8) {
    // Per instruction: 16 rows x 64 contiguous bytes.
#pragma unroll
    for (int c = 0; c < D / 32; ++c) t.k[c] = ld16(krow + (32 * c + 8 * g) * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) ld_words(vrow[i] + (D / 16) * r * 2, t.v[i]);
  } else {
#pragma unroll
    for (int c = 0; c < D / 64; ++c) t.k[c] = ld16(krow + (D / 4) * g + 16 * c);
#pragma unroll
    for (int i = 0; i < 4; ++i) ld_words(vrow[i] + (D / 16) * r, t.v[i]);
  }
}

// ---------------------------------------------------------------------------
// Fused store (fk_store_paged_decode).  Sequence b's new token is at position
// ctx - 1, in the sequence's last tile.  Each wave that streams that tile
// writes its kv head's slice of b's new K/V row to slot_mapping[b] (when in
// range) right before it fetches the tile, and then reads position ctx - 1
// from the cache like any other, as the reference's store-then-decode does: a
// wave's vector memory operations complete in order and its lanes share one
// L1, so its own writes are visible to its later loads.  The row is loaded at
// the start of the segment, so the write does not wait for it.  Every column
// block of a kv head writes the same bytes.  Sequences with no context are
// written by a designated work-group.  A slot that other work-groups read in
// the same launch (one that is not position ctx - 1 of its own sequence) is
// written in no defined order against those reads.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t slot_of(const DecodeParams& P, const void* __restrict__ sm,
                                           int b) {
  return P.slot_is_i64 ? static_cast<const int64_t*>(sm)[b]
                       : static_cast<int64_t>(static_cast<const int32_t*>(sm)[b]);
}

// In-range slot of sequence b's new row, or -1.
__device__ __forceinline__ int64_t valid_slot(const DecodeParams& P, const void* __restrict__ sm,
                                              int b) {
  const int64_t slot = slot_of(P, sm, b);
  return (slot >= 0 && slot < (P.num_blocks << P.block_size_log2)) ? slot : -1;
}

// One 16-byte chunk of sequence b's new K/V row for kv head kvh, in the layout
// store_new_chunk writes: lanes 0..31 hold K chunk (lane & 31), lanes 32..63 V
// chunk (lane & 31); chunk indices past the row re-read a valid chunk and are
// not stored.
template <bool kFp8, int D>
__device__ __forceinline__ uint4 load_new_chunk(const DecodeParams& P, int b, int kvh, int lane) {
  constexpr int kElem = kFp8 ? 1 : 2;
  constexpr int kChunks = D * kElem / 16;
  const int c = min(lane & 31, kChunks - 1);
  const int64_t head_off = static_cast<int64_t>(kvh) * D * kElem;
  const bool is_v = lane >= 32;
  const uint8_t* src = (is_v ? P.new_v + b * P.new_v_stride : P.new_k + b * P.new_k_stride) +
                       head_off + 16 * c;
  return ld16(src);
}
template <bool kFp8, int D>
__device__ __forceinline__ void store_new_chunk(const DecodeParams& P, int64_t slot, int kvh,
                                                int lane, const uint4& v) {
  constexpr int kElem = kFp8 ? 1 : 2;
  constexpr int kChunks = D * kElem / 16;
  const int c = lane & 31;
  if (c >= kChunks) return;
  const int64_t row_bytes = static_cast<int64_t>(P.num_kv_heads) * D * kElem;
  uint8_t* dst = const_cast<uint8_t*>(lane >= 32 ? P.v_cache : P.k_cache) + slot * row_bytes +
                 static_cast<int64_t>(kvh) * D * kElem + 16 * c;
  *reinterpret_cast<uint4*>(dst) = v;
}

// Writes kv head kvh of sequence b's new K and V rows to cache slot `slot`.
template <bool kFp8, int D>
__device__ __forceinline__ void store_new_row(const DecodeParams& P, int b, int kvh, int64_t slot,
                                              int lane) {
  store_new_chunk<kFp8, D>(P, slot, kvh, lane, load_new_chunk<kFp8, D>(P, b, kvh, lane));
}

// ---------------------------------------------------------------------------
// Helpers of the A/B tile forms (FK_DECODE_VALU_TILE, FK_DECODE_LDS_STAGE).
// ---------------------------------------------------------------------------
// DPP row reductions over the 16 lanes of each row: quad_perm [1,0,3,2] and
// [2,3,0,1], then row_half_mirror and row_mirror; every lane gets the result.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  return fmaxf(v, dpp_f<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  return v + dpp_f<0x140>(v);
}
// c + a.lo * b.lo + a.hi * b.hi over bf16 pairs (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const bf16x2_t p = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, p);
}
// Word v of lane src (ds_bpermute).
__device__ __forceinline__ uint32_t lane_word(uint32_t v, int src) {
  return static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src << 2, static_cast<int>(v)));
}
// 16 bytes from global memory straight into LDS: lane l writes at lds_addr +
// 16 l.  Inline asm, so the compiler's wait-count pass does not track it; the
// ring below orders it with explicit s_waitcnt.  M0 carries the LDS address
// and is restored afterwards.
__device__ __forceinline__ void lds_dma16(const uint8_t* src, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_nop 0\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(lds_addr)
      : "memory");
}
__device__ __forceinline__ uint32_t lds_addr_of(const uint8_t* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t*)p));
}
constexpr int kStageBytes = 8192;  // one bf16 tile at head size 128: K 4 KiB, then V 4 KiB

// Online-softmax state of one wave over the query heads of one virtual head,
// and the tile loop that streams a token range [tok_begin, tok_end) of a
// sequence through it (tok_begin a multiple of 16).  Lane (r, g) of the O
// accumulators holds O[column 4g + i][dims (D/16) r .. (D/16) r + D/16 - 1].
template <int kG, int D, bool kFp8, int U, bool kStore>
struct WaveState {
  static constexpr int kKc = D / 32;  // K chunks per row (QK^T MFMAs per tile)
  static constexpr int kSl = D / 16;  // P.V slices; also dims per lane
  // A/B forms (off in the shipped build).
  static constexpr bool kValu = kValuBuild && !kFp8 && D == 128 && kG == 4;
  static constexpr bool kLds = kLdsBuild && !kFp8 && D == 128 && !kStore;
  uint8_t* ring;  // kLds: this wave's two LDS stages
  float m_run;  // running max of column r (same in the 4 lanes of a column)
  float l_run;  // this lane's share of the running sum of column r
  floatx4_t o[kSl];

  // Keys below key_lo (the sliding window's start) are masked; tok_begin is
  // the start of the tile holding key_lo or later.  kStore: a segment that ends
  // at the context end writes b's new row before it fetches the last tile.
  // idle: a wave past the last virtual head; it loads nothing and only keeps
  // the work-group's barrier count.
  // lockstep false: no lock-step barriers (the waves of the work-group stream
  // ranges of different lengths).
  __device__ __forceinline__ void run(const DecodeParams& P, const int32_t* __restrict__ bt,
                                      const void* __restrict__ sm, int b, const VHead& vh,
                                      int tok_begin, int tok_end, int ctx, int key_lo, int r,
                                      int g, bool idle, bool lockstep = true) {
    constexpr int kSyncChunks = kFp8 ? FK_DECODE_SYNC_CHUNKS_FP8 : FK_DECODE_SYNC_CHUNKS;
    constexpr bool kSync = kSyncChunks > 0 && !kLds;
    if (idle) {
      if (kSync && lockstep) {
        const int n = (tok_end - tok_begin + kTile - 1) / kTile;
#pragma unroll 1
        for (int t0 = 0, c = 0; t0 < n; t0 += U, ++c)
          if (c % kSyncChunks == 0) __builtin_amdgcn_s_barrier();
      }
      return;
    }
    const int kvh = vh.kvh;
    uint4 new_chunk = make_uint4(0, 0, 0, 0);  // this lane's chunk of b's new row
    int64_t new_slot = -1;
    int t_store = -1;  // the tile (from tok_begin) holding position ctx - 1
    if constexpr (kStore) {
      if (tok_end == ctx && ctx > tok_begin) {  // wave-uniform
        new_chunk = load_new_chunk<kFp8, D>(P, b, kvh, 16 * g + r);
        new_slot = valid_slot(P, sm, b);
        t_store = (ctx - 1 - tok_begin) / kTile;
      }
    }
    const bool head_ok = r < vh.ncols;
    // kValu: lane (r, g) holds Q[head j][dims 32c + 8g .. +7] of the 4 heads, and
    // (vm, vl) are head j's running max and this lane's share of its sum.
    uint4 qv[kValu ? 4 : 1][kValu ? 4 : 1];
    float vm[4], vl[4];
    if constexpr (kValu) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint16_t* qp = P.q + b * P.q_row_stride + static_cast<int64_t>(vh.qbase + j) * D;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          qv[j][c] = j < vh.ncols ? *reinterpret_cast<const uint4*>(qp + 32 * c + 8 * g)
                                  : make_uint4(0, 0, 0, 0);
        vm[j] = kNegInf;
        vl[j] = 0.f;
      }
    }
    // Q^T operand: column r = query head qbase + r; dims permuted as the K loads.
    bf16x8_t qb[kKc];
    {
      const uint16_t* qp = P.q + b * P.q_row_stride + static_cast<int64_t>(vh.qbase + r) * D;
#pragma unroll
      for (int c = 0; c < kKc; ++c) {
        const int d0 = kFp8 ? (D / 4) * g + 8 * c : 32 * c + 8 * g;
        uint4 v = head_ok ? *reinterpret_cast<const uint4*>(qp + d0) : make_uint4(0, 0, 0, 0);
        qb[c] = __builtin_bit_cast(bf16x8_t, v);
      }
    }
    const float s2 = P.scale_log2;
    // fp8 dequant scales of this kv head (1 for bf16 pages or no scale tensor).
    const float ks = (kFp8 && P.k_scale) ? P.k_scale[kvh] : 1.f;
    const float vsc = (kFp8 && P.v_scale) ? P.v_scale[kvh] : 1.f;

    m_run = kNegInf;
    l_run = 0.f;
#pragma unroll
    for (int d = 0; d < kSl; ++d) o[d] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    // Visible tokens are [key_lo, tok_end): one unsigned compare of tok - key_lo
    // against their count checks both bounds.
    const uint32_t span = static_cast<uint32_t>(tok_end - key_lo);
    // One 16-token tile: scores, online softmax update, P.V accumulation.
    auto process = [&](int tok0, int64_t page, const DTile<kFp8, D>& cur) {
      const int rel0 = tok0 + 4 * g - key_lo;
      if constexpr (kValu) {
        // Scores of token r for the 4 heads: dot products over the lane's 32
        // dims, summed over the 4 lane groups (every lane of row r gets them).
        const bool tok_ok = page >= 0 && static_cast<uint32_t>(tok0 + r - key_lo) < span;
        float pj[4], alpha[4];
        bool moved = false;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float a = 0.f;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            a = dot2_bf16(cur.k[c].x, qv[j][c].x, a);
            a = dot2_bf16(cur.k[c].y, qv[j][c].y, a);
            a = dot2_bf16(cur.k[c].z, qv[j][c].z, a);
            a = dot2_bf16(cur.k[c].w, qv[j][c].w, a);
          }
          a = pair_sum(a);
          const float sj = (tok_ok && j < vh.ncols) ? a * s2 : kNegInf;
          const float m_new = fmaxf(vm[j], row16_max(sj));
          const float m_use = m_new == kNegInf ? 0.f : m_new;
          alpha[j] = m_new == kNegInf ? 1.f : __builtin_amdgcn_exp2f(vm[j] - m_use);
          moved |= alpha[j] != 1.f;
          pj[j] = __builtin_amdgcn_exp2f(sj - m_use);
          vl[j] = vl[j] * alpha[j] + pj[j];
          vm[j] = m_new;
        }
        // o[e][j]: head j, dim 8r + e, summed over this lane's 4 tokens.
        if (__ballot(moved) != 0) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int j = 0; j < 4; ++j) o[e][j] *= alpha[j];
        }
        // P[head j, token 4g + i] from lane 16g + 4g + i (heads packed in
        // pairs), regrouped into token pairs for the dot products.
        const uint32_t w01 = pack_bf16x2(pj[0], pj[1]), w23 = pack_bf16x2(pj[2], pj[3]);
        uint32_t f01[4], f23[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f01[i] = lane_word(w01, 20 * g + i);
          f23[i] = lane_word(w23, 20 * g + i);
        }
        uint32_t pp[4][2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          pp[0][k] = lo_pair(f01[2 * k], f01[2 * k + 1]);
          pp[1][k] = hi_pair(f01[2 * k], f01[2 * k + 1]);
          pp[2][k] = lo_pair(f23[2 * k], f23[2 * k + 1]);
          pp[3][k] = hi_pair(f23[2 * k], f23[2 * k + 1]);
        }
        uint32_t vw[4][D / 32];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v_words(cur, i, page >= 0 && static_cast<uint32_t>(rel0 + i) < span, vw[i]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t v0l = lo_pair(vw[0][q], vw[1][q]), v1l = lo_pair(vw[2][q], vw[3][q]);
          const uint32_t v0h = hi_pair(vw[0][q], vw[1][q]), v1h = hi_pair(vw[2][q], vw[3][q]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            o[2 * q][j] = dot2_bf16(pp[j][1], v1l, dot2_bf16(pp[j][0], v0l, o[2 * q][j]));
            o[2 * q + 1][j] = dot2_bf16(pp[j][1], v1h, dot2_bf16(pp[j][0], v0h, o[2 * q + 1][j]));
          }
        }
        return;
      }
      uint4 kc[kKc];
      k_chunks_d(cur, kc, ks);
      const floatx4_t acc = qk_scores_n(kc, qb);
      // A tile wholly inside the visible keys on a readable page (every tile but
      // those at a segment's edges) needs no mask: one wave-uniform test skips
      // the per-token compares and selects.  Padding columns (r >= ncols) have a
      // zero Q, so their scores stay finite; their rows are never written.
      const bool full = page >= 0 && tok0 >= key_lo && tok0 + kTile <= tok_end;
      float s[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] = acc[i] * s2;
      if (!full) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (!(page >= 0 && static_cast<uint32_t>(rel0 + i) < span)) s[i] = kNegInf;
      }
      float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
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
          for (int d = 0; d < kSl; ++d) o[d][i] *= a;
        }
      }
      const short4_t pa = p_operand(pr);
      // V rows past the context (inside a valid page) may hold anything: zero
      // them so that P = 0 never meets a NaN.
      short4_t vb[kSl];
      if constexpr (kFp8) {
        bool keep[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) keep[i] = page >= 0 && static_cast<uint32_t>(rel0 + i) < span;
        v_operands_fp8(cur, vsc, full, keep, vb);
      } else {
        uint32_t vw[4][D / 32];
#pragma unroll
        for (int i = 0; i < 4; ++i) v_words(cur, i, true, vw[i]);
        if (!full) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool keep = page >= 0 && static_cast<uint32_t>(rel0 + i) < span;
#pragma unroll
            for (int q = 0; q < D / 32; ++q) vw[i][q] = keep ? vw[i][q] : 0u;
          }
        }
        v_operands_w(vw, vb);
      }
      pv_accumulate_n(o, pa, vb);
    };

    const int ntiles = (tok_end - tok_begin + kTile - 1) / kTile;
    // The last block-table entry looked up (wave-uniform): a page holds
    // block_size / 16 tiles, so most tiles reuse it instead of a scalar load.
    int pc_idx = -1;
    int64_t pc_page = -1;
    // Issues the loads of tiles t0 .. t0+U-1 into `buf` (unconditional; tiles
    // past the end re-read the last tile, which hits in cache).
    auto fetch = [&](int t0, DTile<kFp8, D>(&buf)[U], int64_t(&pg)[U]) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int tok0 = tok_begin + kTile * min(t0 + u, ntiles - 1);
        const int idx = tok0 >> P.block_size_log2;
        if (idx != pc_idx) {
          pc_page = page_of(P, bt, b, tok0);
          pc_idx = idx;
        }
        pg[u] = pc_page;
        load_tile<kFp8, D>(P, pg[u] < 0 ? 0 : pg[u], kvh, tok0, r, g, buf[u]);
      }
    };
    auto consume = [&](int t0, const DTile<kFp8, D>(&buf)[U], const int64_t(&pg)[U]) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (t0 + u < ntiles) process(tok_begin + kTile * (t0 + u), pg[u], buf[u]);
      }
    };
    // Chunks of U tiles: issue all U tiles' loads, then consume them in order
    // (the compiler waits for tile u with vmcnt = loads issued after it).
    if constexpr (kLds) {
      run_lds_ring(P, bt, b, kvh, tok_begin, ntiles, r, g, pc_idx, pc_page, process);
    } else {
      for (int t0 = 0, c = 0; t0 < ntiles; t0 += U, ++c) {
        // Lock step (no wait for memory: gfx950's barrier does not drain the
        // loads in flight).
        if constexpr (kSync) {
          if (lockstep && c % kSyncChunks == 0) __builtin_amdgcn_s_barrier();
        }
        if constexpr (kStore) {
          if (t_store >= t0 && t_store < t0 + U && new_slot >= 0)
            store_new_chunk<kFp8, D>(P, new_slot, kvh, 16 * g + r, new_chunk);
        }
        DTile<kFp8, D> buf[U];
        int64_t pg[U];
        fetch(t0, buf, pg);
        consume(t0, buf, pg);
      }
    }
    if constexpr (kValu) {
      // Sum O over the 4 lane groups: lanes of group 0 then hold the MFMA
      // layout (column i = head i), which is what the writers read.
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int j = 0; j < 4; ++j) o[e][j] = pair_sum(o[e][j]);
      float lt[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) lt[j] = row16_sum(vl[j]);
      const int rr = r & 3;
      m_run = rr == 0 ? vm[0] : rr == 1 ? vm[1] : rr == 2 ? vm[2] : vm[3];
      l_run = rr == 0 ? lt[0] : rr == 1 ? lt[1] : rr == 2 ? lt[2] : lt[3];
    } else {
      // Column sums of l over the 4 lane groups: every lane of column j holds l_j.
      l_run = pair_sum(l_run);
    }
  }

  // kLds tile loop: tile t is staged in ring stage t % 2, tile t + 1's 8 loads
  // are issued before tile t is waited for, read from LDS and processed.
  // Tiles past the end re-read the last tile, so every wait is vmcnt(8).
  template <typename Process>
  __device__ __forceinline__ void run_lds_ring(const DecodeParams& P,
                                               const int32_t* __restrict__ bt, int b, int kvh,
                                               int tok_begin, int ntiles, int r, int g,
                                               int& pc_idx, int64_t& pc_page, Process& process) {
    const int lane = 16 * g + r;
    const uint32_t ring_addr = __builtin_amdgcn_readfirstlane(lds_addr_of(ring));
    const int64_t row_bytes = static_cast<int64_t>(P.num_kv_heads) * D * 2;
    const int64_t head_off = static_cast<int64_t>(kvh) * D * 2;
    auto issue = [&](int t, int stage) -> int64_t {
      const int tok0 = tok_begin + kTile * min(t, ntiles - 1);
      const int idx = tok0 >> P.block_size_log2;
      if (idx != pc_idx) {
        pc_page = page_of(P, bt, b, tok0);
        pc_idx = idx;
      }
      const int64_t page = pc_page < 0 ? 0 : pc_page;
      const int64_t slot0 = (page << P.block_size_log2) + (tok0 & ((1 << P.block_size_log2) - 1));
      const uint8_t* krow = P.k_cache + (slot0 + r) * row_bytes + head_off;
      const uint32_t base = ring_addr + stage * kStageBytes;
#pragma unroll
      for (int c = 0; c < 4; ++c) lds_dma16(krow + (32 * c + 8 * g) * 2, base + 1024 * c);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        lds_dma16(P.v_cache + (slot0 + 4 * g + i) * row_bytes + head_off + 16 * r,
                  base + 4096 + 1024 * i);
      return pc_page;
    };
    auto read = [&](int stage, DTile<kFp8, D>& t) {
      const uint8_t* p = ring + stage * kStageBytes + 16 * lane;
#pragma unroll
      for (int c = 0; c < 4; ++c) t.k[c] = *reinterpret_cast<const uint4*>(p + 1024 * c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 x = *reinterpret_cast<const uint4*>(p + 4096 + 1024 * i);
        t.v[i][0] = x.x;
        t.v[i][1] = x.y;
        t.v[i][2] = x.z;
        t.v[i][3] = x.w;
      }
    };
    int64_t pg0 = issue(0, 0), pg1 = -1;
    for (int t = 0; t < ntiles; t += 2) {
      pg1 = issue(t + 1, 1);
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      {
        DTile<kFp8, D> cur;
        read(0, cur);
        process(tok_begin + kTile * t, pg0, cur);
      }
      if (t + 1 >= ntiles) break;
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // stage 0's reads are done
      pg0 = issue(t + 2, 0);
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      {
        DTile<kFp8, D> cur;
        read(1, cur);
        process(tok_begin + kTile * (t + 1), pg1, cur);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // stage 1's reads are done
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring is free for the next segment
  }

  // Normalised output rows of the virtual head for a sequence finished in place.
  __device__ __forceinline__ void write_final(const DecodeParams& P, int b, const VHead& vh,
                                              int r, int g) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * g + i;
      float l = row_value<kG>(l_run, g, i);
      if (P.sinks)
        l = with_sink(l, row_value<kG>(m_run, g, i),
                      sink_log2(P, vh.qbase + (j < vh.ncols ? j : 0)));
      if (j >= kG || j >= vh.ncols) continue;
      const float f = l > 0.f ? 1.f / l : 0.f;
      uint32_t w[D / 32];
#pragma unroll
      for (int d = 0; d < D / 32; ++d) {
        const bf16x2_t pk = {static_cast<__bf16>(o[2 * d][i] * f),
                             static_cast<__bf16>(o[2 * d + 1][i] * f)};
        w[d] = __builtin_bit_cast(uint32_t, pk);
      }
      uint16_t* dst = P.out + b * P.out_row_stride + static_cast<int64_t>(vh.qbase + j) * D +
                      (D / 16) * r;
      if constexpr (D == 64) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
      } else {
#pragma unroll
        for (int q = 0; q < D / 128; ++q)
          *reinterpret_cast<uint4*>(dst + 8 * q) =
              make_uint4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
      }
    }
  }

  // Unnormalised partial (O, and (max, sum)) into partial rows row0 + hq for
  // the virtual head's query heads hq.
  __device__ __forceinline__ void write_partial(const DecodeParams& P, int64_t row0,
                                                const VHead& vh, int r, int g) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * g + i;
      if (j >= kG || j >= vh.ncols) continue;
      float* dst = P.part_o + (row0 + vh.qbase + j) * D + (D / 16) * r;
#pragma unroll
      for (int q = 0; q < kSl / 4; ++q)
        *reinterpret_cast<float4*>(dst + 4 * q) =
            make_float4(o[4 * q][i], o[4 * q + 1][i], o[4 * q + 2][i], o[4 * q + 3][i]);
    }
    if (g == 0 && r < vh.ncols) {
      P.part_ml[(row0 + vh.qbase + r) * 2 + 0] = m_run;
      P.part_ml[(row0 + vh.qbase + r) * 2 + 1] = l_run;
    }
  }
};

// Registers held to what two waves per SIMD leave (256 VGPRs + AGPRs): for a
// work-group of fewer than 8 waves the compiler's own occupancy target would
// let them grow past it (to 272 at head size 256, one wave per SIMD), and the
// plans count on up to 8 resident waves per CU.
#ifndef FK_DECODE_WAVES_PER_EU
#define FK_DECODE_WAVES_PER_EU 2
#endif
// Balanced schedule with fewer than 8 virtual heads (one work-group of fewer
// than 8 waves holds every kv head, and streams its own range): work-groups
// per CU times the kv heads.  A group-count sweep at C3's lengths put the
// optimum at four kv heads' worth per CU (1 kv head: 4 groups; 2: 2; 4: 1):
// Hq 16 / Hk 2 / head 256 122.9 -> 115.7 us, Hq 8 / Hk 1 / head 128 42.6 ->
// 40.4 us, Hq 64 / Hk 2 / head 128 94.3 -> 79.4 us.
#ifndef FK_DECODE_SMALL_WAVES
#define FK_DECODE_SMALL_WAVES 4
#endif

// Fixed partitions: work-group = (partition p, virtual-head group, sequence b);
// wave w owns virtual head blockIdx.y * NH + w and streams the partition.
// Partial rows: (b * max_parts + p) * Hq + hq.
// With P.split = 2 the work-group has 2 NH waves: wave w + NH takes the second
// half of the partition's tiles for the same virtual head, leaves (O, max, sum)
// in LDS (dynamic, split_state_floats per virtual head) and wave w merges it
// with the log-sum-exp rule before writing.  A launch whose fixed partitions
// give one wave per SIMD (C5's 16 partitions: 8 sequences x 16 partitions x 8
// kv heads = 1024 waves) then runs two.
template <int D>
constexpr int split_state_floats() { return (D / 16) * 4 * 64 + 2 * 64; }
template <int NH, int kG, int D, bool kFp8, int U, bool kStore>
__global__ __launch_bounds__(NH < 8 ? 2 * NH * 64 : NH * 64)
__attribute__((amdgpu_waves_per_eu(FK_DECODE_WAVES_PER_EU))) void paged_decode_partition_kernel(
    DecodeParams P, const int32_t* __restrict__ block_tables, const int32_t* __restrict__ ctx_lens,
    const void* __restrict__ slot_mapping) {
  extern __shared__ __align__(16) float split_x[];  // P.split == 2: the second waves' states
  const int p = blockIdx.x;
  const int b = blockIdx.z;
  const int ctx = ctx_lens[b];
  const int tok_begin = p * P.part_tokens;
  // Wave index made provably uniform so that page lookups are scalar loads.
  const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wave = wave_id & (NH - 1);  // the virtual-head slot
  const int sub = wave_id / NH;         // which half of the partition (P.split == 2)
  const int v = blockIdx.y * NH + wave;
  // Waves past the last virtual head only keep the work-group's barrier count.
  const bool idle = v >= P.num_kv_heads * P.col_blocks;  // uniform over the wave
  const VHead vh = vhead(P, idle ? 0 : v);
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
    using WS = WaveState<kG, D, kFp8, U, kStore>;
    WS st;
    __shared__ __align__(16) uint8_t ring[WS::kLds ? NH * 2 * kStageBytes : 16];
    st.ring = ring + wave * 2 * kStageBytes;
    const int seg_begin = max(tok_begin, lo & ~(kTile - 1));
    if (P.split == 1) {
      st.run(P, block_tables, slot_mapping, b, vh, seg_begin, tok_end, ctx, lo, r, g, idle);
    } else {
      // Halves of the partition's tiles (the first takes the odd one); the
      // waves stream different lengths, so no lock-step barriers.
      const int n = max(0, (tok_end - seg_begin + kTile - 1) / kTile);
      const int mid = min(tok_end, seg_begin + ((n + 1) / 2) * kTile);
      st.run(P, block_tables, slot_mapping, b, vh, sub == 0 ? seg_begin : mid,
             sub == 0 ? mid : tok_end, ctx, lo, r, g, idle, false);
      constexpr int kSl = D / 16;
      float* const x = split_x + wave * split_state_floats<D>();
      if (sub == 1 && !idle) {
#pragma unroll
        for (int d = 0; d < kSl; ++d)
          *reinterpret_cast<floatx4_t*>(x + (d * 64 + lane) * 4) = st.o[d];
        x[kSl * 256 + lane] = st.m_run;
        x[kSl * 256 + 64 + lane] = st.l_run;
      }
      __syncthreads();
      if (sub == 1) return;
      if (!idle) {
        // reduce_segments' rule per query column (m, l in column layout; O rows
        // 4g + i take their column's weights): M = max, w = 2^(m - M), 0 for an
        // empty half.
        const float mb = x[kSl * 256 + lane];
        const float lb = x[kSl * 256 + 64 + lane];
        const float ma = st.m_run;
        const float mx = fmaxf(ma, mb);
        const float wa = ma == kNegInf ? 0.f : __builtin_amdgcn_exp2f(ma - mx);
        const float wb = mb == kNegInf ? 0.f : __builtin_amdgcn_exp2f(mb - mx);
        st.m_run = mx;
        st.l_run = st.l_run * wa + lb * wb;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float fa = row_value<kG>(wa, g, i), fb = row_value<kG>(wb, g, i);
#pragma unroll
          for (int d = 0; d < kSl; ++d)
            st.o[d][i] = st.o[d][i] * fa + x[(d * 64 + lane) * 4 + i] * fb;
        }
      }
    }
    if (idle) return;
    if (nparts == 1) {
      st.write_final(P, b, vh, r, g);
    } else {
      const int64_t row0 = (static_cast<int64_t>(b) * P.max_parts + p) * P.num_heads;
      st.write_partial(P, row0, vh, r, g);
    }
  }
  // No partition streams position ctx - 1 (no context): partition 0 writes b's
  // row.
  if (kStore && p == 0 && ctx <= 0 && vh.first && !idle && sub == 0) {
    const int64_t os = valid_slot(P, slot_mapping, b);
    if (os >= 0) store_new_row<kFp8, D>(P, b, vh.kvh, os, lane);
  }
}

// Tiles a sequence of ctx tokens streams: from the tile of its first visible
// key (the sliding window's start) to the end.
__device__ __forceinline__ int tiles_of(const DecodeParams& P, int ctx) {
  return ctx > 0 ? (ctx + kTile - 1) / kTile - key_lo(P, ctx) / kTile : 0;
}

// Balanced schedule: work-group w (of num_groups per virtual-head group) takes
// tiles [w * S, (w+1) * S) of the concatenation of all sequences' tiles,
// S = ceil(total / num_groups).  Partial rows of a cut sequence:
// (w * 2 + slot) * Hq + hq, slot 0 = the group's first segment, slot 1 = its
// last (a group holds at most one cut sequence at each end).
template <int NH, int kG, int D, bool kFp8, int U, bool kStore>
__global__ __launch_bounds__(NH * 64)
__attribute__((amdgpu_waves_per_eu(FK_DECODE_WAVES_PER_EU))) void paged_decode_balanced_kernel(
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
  const int v = blockIdx.y * NH + wave;
  // Waves past the last virtual head only keep the work-group's barrier count.
  const bool idle = v >= P.num_kv_heads * P.col_blocks;  // uniform over the wave
  const VHead vh = vhead(P, idle ? 0 : v);
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
    using WS = WaveState<kG, D, kFp8, U, kStore>;
    WS st;
    __shared__ __align__(16) uint8_t ring[WS::kLds ? NH * 2 * kStageBytes : 16];
    st.ring = ring + wave * 2 * kStageBytes;
    for (int b = lo; b < batch && toff[b] < t_hi; ++b) {
      const int s_lo = max(t_lo, toff[b]) - toff[b];
      const int s_hi = min(t_hi, toff[b + 1]) - toff[b];
      if (s_hi <= s_lo) continue;  // empty sequence
      const int ctx = ctx_lens[b];
      const int klo = key_lo(P, ctx);
      const int t_first = klo / kTile;  // the sequence's tile s is its tile t_first + s
      st.run(P, block_tables, slot_mapping, b, vh, kTile * (t_first + s_lo),
             min(ctx, kTile * (t_first + s_hi)), ctx, klo, r, g, idle);
      if (idle) continue;
      if (toff[b] >= t_lo && toff[b + 1] <= t_hi) {
        st.write_final(P, b, vh, r, g);
      } else {
        const int slot = toff[b] <= t_lo ? 0 : 1;
        const int64_t row0 = (static_cast<int64_t>(w) * 2 + slot) * P.num_heads;
        st.write_partial(P, row0, vh, r, g);
      }
    }
  }
  // Sequences without tiles (no context) have no range that holds their last
  // position: group w writes the rows of those with b = w mod G.
  if (kStore && vh.first && !idle) {
    for (int b = w; b < batch; b += P.num_groups) {
      if (toff[b + 1] != toff[b]) continue;
      const int64_t os = valid_slot(P, slot_mapping, b);
      if (os >= 0) store_new_row<kFp8, D>(P, b, vh.kvh, os, lane);
    }
  }
}

// Merge of one (query head hq, sequence b) by one wave (merge_fold); each lane
// owns D / 64 dims.  The pieces are taken kMergeBatch at a time (one batch for
// up to 64 pieces): lane k loads piece k's (max, sum) while the wave issues the
// O loads of the batch's first merge_unroll<D>() pieces (32 VGPRs of loads, all
// independent; each row's base address is a scalar pair, as the wave's query
// head is uniform), so up to that many pieces (16 at D = 128) cost one load
// latency; the batch max and sum are wave reductions, and a running (M, L, O)
// carries across batches with the reduce_segments rescaling.  A row with more
// pieces than that (a long sequence in a small batch: one sequence over 256
// work-groups leaves 256) takes kWaves / kRows waves, which fold pieces w,
// w + kWaves / kRows, ... each and are combined through LDS (merge_group).
// Three work-group layouts, picked per launch from the pieces a row is
// expected to hold (launch_reduce_d): 4 rows of one wave (few pieces: idle
// waves would only take dispatch slots), 4 rows of 4 waves, 1 row of 16 waves.
constexpr int kMergeBatch = 64;  // pieces per batch: one (max, sum) per lane
constexpr int kMergeRows = 4;    // rows (query heads of one sequence) per work-group
constexpr int kMergeWide = 16;   // waves per work-group of the split layouts
template <int D>
constexpr int merge_unroll() {  // O rows in flight per wave: 32 registers per lane
  return 2048 / D;
}

template <int D>
struct MergeVec {
  static constexpr int N = D / 64;  // dims per lane
  float x[N];
  __device__ __forceinline__ static MergeVec load(const float* p) {
    MergeVec v;
    if constexpr (N == 1) {
      v.x[0] = *p;
    } else if constexpr (N == 2) {
      const float2 t = *reinterpret_cast<const float2*>(p);
      v.x[0] = t.x;
      v.x[1] = t.y;
    } else {
      const float4 t = *reinterpret_cast<const float4*>(p);
      v.x[0] = t.x;
      v.x[1] = t.y;
      v.x[2] = t.z;
      v.x[3] = t.w;
    }
    return v;
  }
  __device__ __forceinline__ static MergeVec zero() {
    MergeVec v;
#pragma unroll
    for (int e = 0; e < N; ++e) v.x[e] = 0.f;
    return v;
  }
};

// Running log-sum-exp state of a merge: max M and sum L (the same in every
// lane) and this lane's D / 64 dims of the unnormalised O.
template <int D>
struct MergeState {
  float M, L;
  float acc[D / 64];
};

// Folds pieces k = 0 .. nrows - 1 (partial row row_of(k)) into a fresh state.
template <int D, class RowOf>
__device__ __forceinline__ MergeState<D> merge_fold(const float* part_o, const float* part_ml,
                                                    RowOf row_of, int nrows, int lane) {
  using V = MergeVec<D>;
  constexpr int N = V::N;
  constexpr int kMergeUnroll = merge_unroll<D>();
  float M = kNegInf, L = 0.f;
  float acc[N];
#pragma unroll
  for (int e = 0; e < N; ++e) acc[e] = 0.f;
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
    V ov[kMergeUnroll];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u)
      ov[u] = u < n ? V::load(part_o + row_of(k0 + u) * D + N * lane) : V::zero();
    const float mb = wave_max(m);
    const float mn = fmaxf(M, mb);
    if (mn == kNegInf) continue;  // no valid piece yet (all rows empty)
    const float a = __builtin_amdgcn_exp2f(M - mn);  // 0 when M = -inf
    const float f = __builtin_amdgcn_exp2f(m - mn);  // lane k's weight; 0 for empty pieces
    L = L * a + wave_sum(l * f);
#pragma unroll
    for (int e = 0; e < N; ++e) acc[e] *= a;
    for (int u0 = 0; u0 < n; u0 += kMergeUnroll) {
      if (u0 > 0) {
#pragma unroll
        for (int u = 0; u < kMergeUnroll; ++u)
          ov[u] = u0 + u < n ? V::load(part_o + row_of(k0 + u0 + u) * D + N * lane) : V::zero();
      }
#pragma unroll
      for (int u = 0; u < kMergeUnroll; ++u) {
        const float wgt = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), min(u0 + u, 63)));
        if (u0 + u < n) {
#pragma unroll
          for (int e = 0; e < N; ++e) acc[e] = __builtin_fmaf(ov[u].x[e], wgt, acc[e]);
        }
      }
    }
    M = mn;
  }
  MergeState<D> st;
  st.M = M;
  st.L = L;
#pragma unroll
  for (int e = 0; e < N; ++e) st.acc[e] = acc[e];
  return st;
}

// Normalised bf16 row from a merged state; the sink joins the row once.
template <int D>
__device__ __forceinline__ void merge_write(uint16_t* orow, const MergeState<D>& st, float sink2,
                                            int lane) {
  constexpr int N = D / 64;
  const float L = with_sink(st.L, st.M, sink2);
  const float inv = L > 0.f ? 1.f / L : 0.f;
  if constexpr (N == 1) {
    orow[lane] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(st.acc[0] * inv));
  } else {
    uint32_t w[N / 2];
#pragma unroll
    for (int e = 0; e < N / 2; ++e) {
      const bf16x2_t pk = {static_cast<__bf16>(st.acc[2 * e] * inv),
                           static_cast<__bf16>(st.acc[2 * e + 1] * inv)};
      w[e] = __builtin_bit_cast(uint32_t, pk);
    }
    if constexpr (N == 2)
      reinterpret_cast<uint32_t*>(orow)[lane] = w[0];
    else
      reinterpret_cast<uint2*>(orow)[lane] = make_uint2(w[0], w[1]);
  }
}

// The merge rows of one work-group: query heads hq0 .. hq0 + kRows - 1 of one
// sequence, all with the same piece count nrows (the pieces of a sequence are
// the same for every head).  Partial row of piece k of head hq: k = 0 is
// alt0 + hq, k >= 1 is first0 + hq + k * row_stride.  Up to merge_unroll<D>()
// pieces (or with one wave per row), wave r merges row r alone; more pieces
// take kSplit = kWaves / kRows waves per row (wave w folds pieces w,
// w + kSplit, ...), whose states wave 0 of the row combines from LDS with the
// same rescaling.  nrows is uniform over the work-group, so every wave meets
// the barrier or none does.
template <int D, int kRows, int kWaves>
__device__ __forceinline__ void merge_group(const DecodeParams& P, uint16_t* out_b, int hq0,
                                            int64_t first0, int64_t alt0, int64_t row_stride,
                                            int nrows, int wave, int lane) {
  constexpr int N = D / 64;
  constexpr int kSplit = kWaves / kRows;
  constexpr int kSlot = 2 + 64 * N;  // floats per wave in LDS: M, L, O
  __shared__ float xs[kSplit > 1 ? kWaves * kSlot : 1];
  if (kSplit == 1 || nrows <= merge_unroll<D>()) {
    const int hq = hq0 + wave;
    if (wave >= kRows || hq >= P.num_heads) return;
    auto row_of = [&](int k) -> int64_t {
      return k == 0 ? alt0 + hq : first0 + hq + k * row_stride;
    };
    merge_write<D>(out_b + static_cast<int64_t>(hq) * D,
                   merge_fold<D>(P.part_o, P.part_ml, row_of, nrows, lane), sink_log2(P, hq),
                   lane);
    return;
  }
  const int r = wave / kSplit;
  const int part = wave - r * kSplit;
  const int hq = hq0 + r;
  const bool valid = hq < P.num_heads;
  auto row_of = [&](int j) -> int64_t {
    const int k = part + kSplit * j;
    return k == 0 ? alt0 + hq : first0 + hq + k * row_stride;
  };
  const int mine = valid && nrows > part ? (nrows - part + kSplit - 1) / kSplit : 0;
  const MergeState<D> st = merge_fold<D>(P.part_o, P.part_ml, row_of, mine, lane);
  float* x = xs + wave * kSlot;
  if (lane == 0) {
    x[0] = st.M;
    x[1] = st.L;
  }
#pragma unroll
  for (int e = 0; e < N; ++e) x[2 + e * 64 + lane] = st.acc[e];
  __syncthreads();
  if (part != 0 || !valid) return;
  const float* xr = xs + r * kSplit * kSlot;
  float M = kNegInf;
#pragma unroll
  for (int v = 0; v < kSplit; ++v) M = fmaxf(M, xr[v * kSlot]);
  MergeState<D> out;
  out.M = M;
  out.L = 0.f;
#pragma unroll
  for (int e = 0; e < N; ++e) out.acc[e] = 0.f;
  if (M != kNegInf) {
#pragma unroll
    for (int v = 0; v < kSplit; ++v) {
      const float mv = xr[v * kSlot];
      const float f = mv == kNegInf ? 0.f : __builtin_amdgcn_exp2f(mv - M);
      out.L += xr[v * kSlot + 1] * f;
#pragma unroll
      for (int e = 0; e < N; ++e) out.acc[e] += xr[v * kSlot + 2 + e * 64 + lane] * f;
    }
  }
  merge_write<D>(out_b + static_cast<int64_t>(hq) * D, out, sink_log2(P, hq), lane);
}

// Zero row of D bf16 for an empty sequence (one wave; each lane D / 64 dims).
template <int D>
__device__ __forceinline__ void zero_row(uint16_t* orow, int lane) {
#pragma unroll
  for (int e = 0; e < D / 64; ++e) orow[(D / 64) * lane + e] = 0;
}

// Fixed partitions: merge sequences with more than one partition; zero empty ones.
// Work-group = kRows query heads blockIdx.x * kRows .. of sequence blockIdx.y
// (merge_group).
template <int D, int kRows, int kWaves>
__global__ __launch_bounds__(kWaves * 64) void paged_decode_partition_reduce_kernel(
    DecodeParams P) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hq0 = blockIdx.x * kRows;
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int ctx = P.ctx_lens[b];
  uint16_t* out_b = P.out + b * P.out_row_stride;
  if (ctx <= 0) {
    if (wave < kRows && hq0 + wave < P.num_heads)
      zero_row<D>(out_b + static_cast<int64_t>(hq0 + wave) * D, lane);
    return;
  }
  const int nparts = min((ctx + P.part_tokens - 1) / P.part_tokens, P.max_parts);
  if (nparts <= 1) return;  // written by the partition kernel
  const int64_t first = static_cast<int64_t>(b) * P.max_parts * P.num_heads;
  merge_group<D, kRows, kWaves>(P, out_b, hq0, first, first, P.num_heads, nparts, wave, lane);
}

// Balanced schedule: merge sequences cut across work-groups; zero empty ones.
// Work-group as the partition reduce.
template <int D, int kRows, int kWaves>
__global__ __launch_bounds__(kWaves * 64) void paged_decode_balanced_reduce_kernel(
    DecodeParams P) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hq0 = blockIdx.x * kRows;
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  uint16_t* out_b = P.out + b * P.out_row_stride;
  const int t0 = P.tile_off[b];
  const int t1 = P.tile_off[b + 1];
  const int S = P.tile_off[P.batch + 1];
  if (t1 <= t0) {
    if (wave < kRows && hq0 + wave < P.num_heads)
      zero_row<D>(out_b + static_cast<int64_t>(hq0 + wave) * D, lane);
    return;
  }
  const int w0 = t0 / S;
  const int w1 = (t1 - 1) / S;
  if (w0 == w1) return;  // finished in place by work-group w0
  const int64_t hqn = P.num_heads;
  // Group w0 holds the sequence in slot 1 unless the sequence starts its range;
  // groups w0+1 .. w1 hold it in slot 0.
  const int slot0 = t0 > w0 * S ? 1 : 0;
  const int64_t first_alt = (static_cast<int64_t>(w0) * 2 + slot0) * hqn;
  const int64_t first = (static_cast<int64_t>(w0) * 2 + 0) * hqn;
  merge_group<D, kRows, kWaves>(P, out_b, hq0, first, first_alt, 2 * hqn, w1 - w0 + 1, wave,
                                lane);
}

// Tuning knobs (compile-time): tiles per load set for bf16 pages at head sizes
// up to 128 (at 256 a tile's loads fill as many registers as two tiles do at
// 128, so one), and for fp8 pages.  At head size 64, four tiles per set
// measured +2% on 20 kv heads and -2% on 8 (C3's lengths), so two.
#ifndef FK_DECODE_CHUNK
#define FK_DECODE_CHUNK 2
#endif
#ifndef FK_DECODE_CHUNK_FP8
#define FK_DECODE_CHUNK_FP8 2
#endif
template <int D, bool kFp8>
constexpr int chunk_tiles() {
  return D >= 256 ? 1 : kFp8 ? FK_DECODE_CHUNK_FP8 : FK_DECODE_CHUNK;
}
constexpr int kMaxWavesPerGroup = 8;     // virtual heads (waves) per work-group
constexpr int kPartQuant = 64;           // fixed-partition granularity in tokens
constexpr int kMaxBalancedBatch = 8192;  // tile prefix sums live in LDS


// Waves per kv head (column blocks of up to 16 query heads) and virtual heads.
int col_blocks(int num_heads, int num_kv_heads) {
  return (num_heads / num_kv_heads + 15) / 16;
}
int virtual_heads(int num_heads, int num_kv_heads) {
  return num_kv_heads * col_blocks(num_heads, num_kv_heads);
}
int waves_per_group(int vheads) {
  return vheads < kMaxWavesPerGroup ? vheads : kMaxWavesPerGroup;
}

// Workspace layout: part_o rows of head_size floats, part_ml rows (256-byte
// aligned), then (balanced only) batch + 2 int32 for the tile prefix sums and
// the range size.
int64_t o_region(int64_t rows, int head_size) {
  return (rows * head_size * 4 + 255) / 256 * 256;
}
int64_t ml_region(int64_t rows) { return (rows * 2 * 4 + 255) / 256 * 256; }

int64_t partial_rows(bool balanced, int64_t batch, int num_heads, int64_t max_parts) {
  // balanced: max_parts = work-groups per virtual-head group, 2 slots each.
  return balanced ? max_parts * 2 * num_heads : batch * num_heads * max_parts;
}

int64_t workspace_bytes(bool balanced, int64_t batch, int num_heads, int head_size,
                        int64_t max_parts) {
  const int64_t rows = partial_rows(balanced, batch, num_heads, max_parts);
  return o_region(rows, head_size) + ml_region(rows) + (balanced ? (batch + 2) * 4 : 0);
}

bool supported_head(int head_size) {
  return head_size == 64 || head_size == 128 || head_size == 256;
}

int validate(const char* name, int64_t batch, int num_heads, int num_kv_heads, int head_size,
             int64_t part_tokens, int64_t max_parts) {
  FK_REQUIRE(batch >= 0 && batch <= 65535, "%s: batch %lld out of range [0, 65535]", name,
             (long long)batch);
  FK_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             "%s: num_heads %d must be a positive multiple of num_kv_heads %d", name, num_heads,
             num_kv_heads);
  if (!supported_head(head_size))
    return set_error(FK_ERR_UNSUPPORTED, "%s: head_size %d unsupported (64, 128 or 256)", name,
                     head_size);
  const int vh = virtual_heads(num_heads, num_kv_heads);
  FK_REQUIRE((vh + kMaxWavesPerGroup - 1) / kMaxWavesPerGroup <= 65535,
             "%s: %d kv heads x %d column blocks exceed the grid", name, num_kv_heads,
             col_blocks(num_heads, num_kv_heads));
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
  int head_size;
  dim3 grid;
  size_t part_lds = 0;  // fixed partitions split over two waves: the merge area
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
  const int64_t need = workspace_bytes(balanced, batch, num_heads, head_size, max_parts);
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
  P.num_heads = num_heads;
  P.num_kv_heads = num_kv_heads;
  P.gqa = num_heads / num_kv_heads;
  P.col_blocks = col_blocks(num_heads, num_kv_heads);
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
  P.part_ml = needs_ws ? reinterpret_cast<float*>(ws + o_region(rows, head_size)) : nullptr;
  P.tile_off = balanced ? reinterpret_cast<int32_t*>(ws + o_region(rows, head_size) +
                                                     ml_region(rows))
                        : nullptr;
  L.balanced = balanced;
  L.fp8 = kv_dtype == FK_DTYPE_FP8_E4M3FN;
  L.head_size = head_size;
  const int vh = virtual_heads(num_heads, num_kv_heads);
  L.nh = waves_per_group(vh);
  if (!balanced) {
    // Fixed partitions: while the grid holds fewer work-groups than CUs (few
    // partitions of a small batch), fewer virtual heads per work-group (a
    // power of two, as the launches take) and more work-groups.
    while (L.nh > 1 && static_cast<int64_t>(max_parts) * batch * ((vh + L.nh - 1) / L.nh) <
                           num_cus()) {
      int p2 = 1;
      while (2 * p2 < L.nh) p2 *= 2;
      L.nh = p2;
    }
  }
  // Fixed partitions that would run one wave per SIMD (or fewer) split each
  // partition over two waves of the work-group.
  P.split = 1;
  if (!balanced && L.nh <= 4 &&
      static_cast<int64_t>(max_parts) * batch * vh < 2LL * 4 * num_cus()) {
    P.split = 2;
    L.part_lds = static_cast<size_t>(L.nh) * (head_size / 16 * 4 * 64 + 2 * 64) * sizeof(float);
  }
  const unsigned hgroups = static_cast<unsigned>((vh + L.nh - 1) / L.nh);
  L.grid = balanced ? dim3(static_cast<unsigned>(max_parts), hgroups, 1)
                    : dim3(static_cast<unsigned>(max_parts), hgroups, static_cast<unsigned>(batch));
  return FK_OK;
}

template <int NH, int G, int D, bool FP8, bool ST>
void launch_main_st(const Launch& L, hipStream_t stream) {
  constexpr int U = chunk_tiles<D, FP8>();
  if (L.balanced) {
    const size_t lds = static_cast<size_t>(L.P.batch + 1) * sizeof(int32_t);
    hipLaunchKernelGGL((paged_decode_balanced_kernel<NH, G, D, FP8, U, ST>), L.grid,
                       dim3(NH * 64), lds, stream, L.P, L.P.block_tables, L.P.ctx_lens,
                       L.slot_mapping);
  } else {
    hipLaunchKernelGGL((paged_decode_partition_kernel<NH, G, D, FP8, U, ST>), L.grid,
                       dim3(NH * L.P.split * 64), L.part_lds, stream, L.P, L.P.block_tables,
                       L.P.ctx_lens, L.slot_mapping);
  }
}

template <int NH, int G, int D, bool FP8>
void launch_main(const Launch& L, hipStream_t stream) {
  if (L.P.new_k != nullptr)
    launch_main_st<NH, G, D, FP8, true>(L, stream);
  else
    launch_main_st<NH, G, D, FP8, false>(L, stream);
}

template <int G, int D, bool FP8>
void launch_main_nh(const Launch& L, hipStream_t stream) {
  switch (L.nh) {
    case 1: launch_main<1, G, D, FP8>(L, stream); break;
    case 2: launch_main<2, G, D, FP8>(L, stream); break;
    case 4: launch_main<4, G, D, FP8>(L, stream); break;
    default: launch_main<8, G, D, FP8>(L, stream); break;
  }
}

template <int G, int D>
void launch_main_gd(const Launch& L, hipStream_t stream) {
  if (L.fp8)
    launch_main_nh<G, D, true>(L, stream);
  else
    launch_main_nh<G, D, false>(L, stream);
}

template <int D>
void launch_main_d(const Launch& L, hipStream_t stream) {
  // Query columns per wave: the group size, rounded up to 4, 8 or 16 (groups
  // above 16 take several 16-column waves per kv head).
  if (L.P.gqa <= 4)
    launch_main_gd<4, D>(L, stream);
  else if (L.P.gqa <= 8)
    launch_main_gd<8, D>(L, stream);
  else
    launch_main_gd<16, D>(L, stream);
}

void launch_main_any(const Launch& L, hipStream_t stream) {
  switch (L.head_size) {
    case 64: launch_main_d<64>(L, stream); break;
    case 256: launch_main_d<256>(L, stream); break;
    default: launch_main_d<128>(L, stream); break;
  }
}

template <int D, int kRows, int kWaves>
void launch_reduce_rows(const Launch& L, int64_t batch, int num_heads, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((num_heads + kRows - 1) / kRows),
                  static_cast<unsigned>(batch));
  if (L.balanced)
    hipLaunchKernelGGL((paged_decode_balanced_reduce_kernel<D, kRows, kWaves>), grid,
                       dim3(kWaves * 64), 0, stream, L.P);
  else
    hipLaunchKernelGGL((paged_decode_partition_reduce_kernel<D, kRows, kWaves>), grid,
                       dim3(kWaves * 64), 0, stream, L.P);
}

// Merge layout from the pieces a row is expected to hold (balanced: about
// ranges / batch + 1 per sequence; fixed partitions: max_parts): one wave per
// row when one wave folds them in one round, four waves per row up to four
// rounds' worth, else a work-group of 16 waves per row.  Every layout merges any
// piece count; this only picks the faster one for the batch.
template <int D>
void launch_reduce_d(const Launch& L, int64_t batch, int num_heads, hipStream_t stream) {
  const int64_t pieces = L.balanced ? (L.P.max_parts + batch - 1) / batch + 1 : L.P.max_parts;
  const int64_t round = merge_unroll<D>();
  if (pieces <= round)
    launch_reduce_rows<D, kMergeRows, kMergeRows>(L, batch, num_heads, stream);
  else if (pieces <= (kMergeWide / kMergeRows) * round)
    launch_reduce_rows<D, kMergeRows, kMergeWide>(L, batch, num_heads, stream);
  else
    launch_reduce_rows<D, 1, kMergeWide>(L, batch, num_heads, stream);
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
                 num_splits >= 0 && num_heads % num_kv_heads == 0,
             "fk_paged_decode_plan: invalid argument");
  if (!supported_head(head_size))
    return set_error(FK_ERR_UNSUPPORTED,
                     "fk_paged_decode_plan: head_size %d unsupported (64, 128 or 256)",
                     head_size);
  const int64_t L = max_seq_len > 0 ? max_seq_len : 1;
  const int vh = virtual_heads(num_heads, num_kv_heads);
  if (num_splits == 0 && batch <= kMaxBalancedBatch) {
    // Balanced: one work-group per CU when one group of 8 virtual heads covers
    // them all; with several full groups, one work-group per CU over all the
    // groups together (a group count that does not divide evenly, or a last
    // group with idle waves, keeps one per CU per group).  Fewer than 8
    // virtual heads make one group of all the kv heads: FK_DECODE_SMALL_WAVES /
    // num_kv_heads work-groups per CU (at least one).
    const int nh = waves_per_group(vh);
    const int hgroups = (vh + nh - 1) / nh;
    const int64_t cus = num_cus();
    *part_tokens = 0;
    if (nh < kMaxWavesPerGroup) {
      const int per = FK_DECODE_SMALL_WAVES / num_kv_heads;
      *max_parts = cus * (per > 1 ? per : 1);
    } else if (hgroups > 1 && vh % kMaxWavesPerGroup == 0 && cus % hgroups == 0) {
      *max_parts = cus / hgroups;
    } else {
      *max_parts = cus;
    }
  } else {
    int64_t part;
    if (num_splits > 0) {
      part = (L + num_splits - 1) / num_splits;
    } else {
      // ~8192 waves (one per (sequence, virtual head, partition)), >= 256 tokens each.
      const int64_t units = (batch > 0 ? batch : 1) * vh;
      part = (L * units + 8191) / 8192;
      if (part < 256) part = 256;
    }
    part = (part + kPartQuant - 1) / kPartQuant * kPartQuant;
    *part_tokens = part;
    *max_parts = (L + part - 1) / part;
  }
  *workspace_bytes_out =
      batch > 0 ? workspace_bytes(*part_tokens == 0, batch, num_heads, head_size, *max_parts) : 0;
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
  launch_main_any(L, as_stream(stream));
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
  hipStream_t s = as_stream(stream);
  switch (head_size) {
    case 64: launch_reduce_d<64>(L, batch, num_heads, s); break;
    case 256: launch_reduce_d<256>(L, batch, num_heads, s); break;
    default: launch_reduce_d<128>(L, batch, num_heads, s); break;
  }
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
  const int64_t row = static_cast<int64_t>(num_kv_heads) * head_size;
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
  launch_main_any(L, as_stream(stream));
  rc = check_launch(name);
  if (rc != FK_OK) return rc;
  return fk_paged_decode_reduce(out, out_row_stride, q, q_row_stride, k_cache, v_cache, kv_dtype,
                                k_scale, v_scale, block_tables, bt_row_stride, ctx_lens, batch,
                                num_heads, num_kv_heads, head_size, block_size, num_blocks, scale,
                                window_left, sinks, part_tokens, max_parts, workspace, ws_bytes,
                                stream);
}
