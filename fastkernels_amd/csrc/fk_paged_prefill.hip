// Paged prefill attention (variable-length query chunks over a paged KV cache)
// for MI355X (gfx950).
//
// Semantics: FlashAttnPrefill.forward with a block table
// (fastkernels/tasks/baseline/L1/flash_attn_prefill.py:28-74: flash_attn_varlen_func
// with cu_seqlens_q, seqused_k = cu_seqlens_k[1:] - cu_seqlens_k[:-1], causal), and
// the reference's torch fallback Attention._prefill_torch_from_cache
// (fastkernels/tasks/baseline/L2/attention_impl.py:640-652, _sdpa_one :606-622):
// sequence b owns query rows [cu_q[b], cu_q[b+1]) (q_len of them) and the first
// k_len = cu_k[b+1] - cu_k[b] tokens of its paged cache.  Query j (0-based in
// its chunk) sits at position k_len - q_len + j and sees keys
// [0, k_len - q_len + j] (causal, aligned to the end of the keys).  A query
// with no visible key gets a zero row.  kv head = hq / (Hq / Hk); fp8 pages
// are dequantised per kv head as in the decode kernel.
//
// Work decomposition: work-group = (block of 32 query tokens, kv head,
// sequence), one wave per query head of the kv head's group (groups above 8
// heads span two work-groups), so the group's waves stream the same K/V tiles
// (shared through L1/L2).  A wave keeps two
// 16-query column blocks of one head in MFMA tiles (fk_attn_tile.h: S = K Q^T
// per 16-key tile, online softmax per query column, O += P V) and walks the
// key tiles up to its last visible key.  The blocks with the most keys (the
// last ones of a sequence) are dispatched first.
#include <type_traits>

#include "fk_attn_tile.h"

namespace fk {
namespace {

#ifndef FK_PREFILL_COLS
#define FK_PREFILL_COLS 2
#endif
#ifndef FK_PREFILL_PREFETCH
#define FK_PREFILL_PREFETCH 1
#endif
// Two waves per SIMD: with the register double buffer the compiler would
// otherwise settle at one (262 registers), and the causal schedule's longest
// work-groups are latency-bound.  Measured on MI355X: 155 us for a 2048-token
// Qwen3-8B prompt against 178-277 us for the other register/occupancy points.
#ifndef FK_PREFILL_WAVES
#define FK_PREFILL_WAVES __attribute__((amdgpu_waves_per_eu(2)))
#endif
#ifndef FK_PREFILL_CHUNK
#define FK_PREFILL_CHUNK 1
#endif
#ifndef FK_PREFILL_LAZY
#define FK_PREFILL_LAZY 8.0f
#endif
constexpr int kColBlocks = FK_PREFILL_COLS;    // 16-query column blocks per wave
constexpr float kLazy = FK_PREFILL_LAZY;       // max-update threshold (log2 units)
constexpr int kChunk = FK_PREFILL_CHUNK;       // key tiles loaded together
constexpr int kQTokens = 16 * kColBlocks;      // query tokens per work-group

struct PrefillParams {
  uint16_t* out;
  int64_t out_row_stride;
  const uint16_t* q;
  int64_t q_row_stride;
  const uint8_t* k_cache;  // paged: the caches; dense: the first key / value row
  const uint8_t* v_cache;
  int64_t k_row_bytes;     // bytes between key rows (paged: Hk * 128 * elem)
  int64_t v_row_bytes;
  const float* k_scale;
  const float* v_scale;
  int64_t bt_row_stride;
  int num_kv_heads;
  int gqa;
  int block_size_log2;
  int64_t num_blocks;
  float scale_log2;
  int causal;  // 0: every query sees all k_len keys
};

__device__ __forceinline__ int64_t prefill_page(const PrefillParams& P,
                                                const int32_t* __restrict__ bt_row, int tok) {
  const int idx = tok >> P.block_size_log2;
  if (idx >= P.bt_row_stride) return -1;
  const int64_t page = bt_row[idx];
  return (page >= 0 && page < P.num_blocks) ? page : -1;
}

// Issues the loads of the 16 key rows starting at row index row0 (a tile never
// spans pages, so its rows are consecutive in both layouts).  Rows above
// row_cap (past the end of a dense key tensor) re-read row_cap; they are masked.
template <bool kFp8>
__device__ __forceinline__ void prefill_load_tile(const PrefillParams& P, int64_t row0,
                                                  int64_t row_cap, int h, int r, int g,
                                                  TileRegs<kFp8>& t) {
  constexpr int kElem = kFp8 ? 1 : 2;
  const int64_t head_off = static_cast<int64_t>(h) * kHead * kElem;
  const uint8_t* krow = P.k_cache + min(row0 + r, row_cap) * P.k_row_bytes + head_off;
  const uint8_t* vbase = P.v_cache + head_off;
  int64_t vr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) vr[i] = min(row0 + 4 * g + i, row_cap);
  if constexpr (!kFp8) {
#pragma unroll
    for (int c = 0; c < 4; ++c) t.k[c] = ld16(krow + (32 * c + 8 * g) * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) t.v[i] = ld16(vbase + vr[i] * P.v_row_bytes + 8 * r * 2);
  } else {
    t.k[0] = ld16(krow + 32 * g);
    t.k[1] = ld16(krow + 32 * g + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) t.v[i] = ld8(vbase + vr[i] * P.v_row_bytes + 8 * r);
  }
}

// Row index of key `tok` of the sequence and whether it is readable: paged, the
// slot through the block table (-1 pages masked; page 0 is read instead);
// dense, row k_start + tok of the key/value tensors.
template <bool kPaged>
__device__ __forceinline__ int64_t key_row(const PrefillParams& P,
                                           const int32_t* __restrict__ bt_row, int k_start,
                                           int tok, bool& ok) {
  if constexpr (kPaged) {
    const int64_t page = prefill_page(P, bt_row, tok);
    ok = page >= 0;
    return ((page < 0 ? 0 : page) << P.block_size_log2) + (tok & ((1 << P.block_size_log2) - 1));
  } else {
    ok = true;
    return static_cast<int64_t>(k_start) + tok;
  }
}

template <int NW, bool kFp8, bool kPaged>
__global__ __launch_bounds__(NW * 64) FK_PREFILL_WAVES void paged_prefill_kernel(
    PrefillParams P, const int32_t* __restrict__ block_tables,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k) {
  const int b = blockIdx.z;
  // Groups of more than 8 query heads per kv head span hsplit work-groups.
  const int hsplit = (P.gqa + NW - 1) / NW;
  const int h = blockIdx.y / hsplit;
  const int head0 = (blockIdx.y - h * hsplit) * NW;  // first query head (within the group)
  const int q_start = cu_q[b];
  const int q_len = cu_q[b + 1] - q_start;
  const int k_start = cu_k[b];
  const int k_len = cu_k[b + 1] - k_start;
  // Heaviest blocks (most keys) first.
  const int qblk = static_cast<int>(gridDim.x) - 1 - static_cast<int>(blockIdx.x);
  const int j0 = qblk * kQTokens;
  if (j0 >= q_len) return;  // uniform over the work-group
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (head0 + wave >= P.gqa) return;
  const int hq = h * P.gqa + head0 + wave;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  // Position of query 0; non-causal, every query sits past the last key.
  const int offset = P.causal ? k_len - q_len : k_len;
  // Keys [0, kend) cover every query of this block.
  const int kend = max(0, min(k_len, offset + min(j0 + kQTokens, q_len)));
  const int32_t* bt_row = kPaged ? block_tables + static_cast<int64_t>(b) * P.bt_row_stride
                                 : nullptr;
  // Dense keys: rows past the sequence's last key would run off the tensor.
  const int64_t row_cap = kPaged ? INT64_MAX : static_cast<int64_t>(k_start) + max(k_len, 1) - 1;

  // Q^T operands: column r of block nb = query j0 + 16 nb + r.
  bf16x8_t qb[kColBlocks][4];
#pragma unroll
  for (int nb = 0; nb < kColBlocks; ++nb) {
    const int j = j0 + 16 * nb + r;
    const bool ok = j < q_len;
    const uint16_t* qp = P.q + static_cast<int64_t>(q_start + (ok ? j : 0)) * P.q_row_stride +
                         static_cast<int64_t>(hq) * kHead;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d0 = kFp8 ? 32 * g + 8 * c : 32 * c + 8 * g;
      const uint4 v = ok ? *reinterpret_cast<const uint4*>(qp + d0) : make_uint4(0, 0, 0, 0);
      qb[nb][c] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  float s2 = P.scale_log2;
  if (kFp8 && P.k_scale) s2 *= P.k_scale[h];

  float m_run[kColBlocks], l_run[kColBlocks];
  floatx4_t o[kColBlocks][8];
#pragma unroll
  for (int nb = 0; nb < kColBlocks; ++nb) {
    m_run[nb] = kNegInf;
    l_run[nb] = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) o[nb][d] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  }

  const int ntiles = (kend + kTile - 1) / kTile;
  // Tiles every query of the block sees in full need no mask: keys up to
  // offset + j0 (query j0's last key), inside [0, kend).
  const int nfull = max(0, min(kend, offset + j0 + 1)) / kTile;

  // One 16-key tile: scores, online softmax per query column, P.V.  kMasked
  // applies the causal / length / page mask; unmasked tiles skip it (every
  // score is finite there, so the running max never stays -inf).
  auto tile_step = [&](auto masked, int tok0, const TileRegs<kFp8>& cur, bool page_ok) {
    constexpr bool kMasked = decltype(masked)::value;
    uint4 kc[4];
    k_chunks(cur, kc);
    uint4 vr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vr[i] = (!kMasked || (page_ok && tok0 + 4 * g + i < kend)) ? v_row(cur, i)
                                                                 : make_uint4(0, 0, 0, 0);
    short4_t vb[8];  // shared by the column blocks
    v_operands(vr, vb);
#pragma unroll
    for (int nb = 0; nb < kColBlocks; ++nb) {
      const floatx4_t acc = qk_scores(kc, qb[nb]);
      const int j = j0 + 16 * nb + r;  // this lane's query column
      const int last = offset + j;     // its last visible key
      float s[4];
      float mt = kNegInf;
      if constexpr (kMasked) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = tok0 + 4 * g + i;
          const bool ok = page_ok && j < q_len && key <= last && key < kend;
          s[i] = ok ? acc[i] * s2 : kNegInf;
          mt = fmaxf(mt, s[i]);
        }
      } else {
        // s2 > 0: the max of the scaled scores is the scaled max.
        mt = fmaxf(fmaxf(acc[0], acc[1]), fmaxf(acc[2], acc[3])) * s2;
      }
      mt = pair_max(mt);
      // Lazy rescaling: the running max only moves when a score exceeds it by
      // more than kLazy (log2 units), so P <= 2^kLazy and the O/l rescale (a
      // cross-lane fetch per row) is rare after the first tiles.  The final
      // normalisation divides by l accumulated against the same max, so the
      // result is unchanged up to rounding.
      const float m_new = mt > m_run[nb] + kLazy ? mt : m_run[nb];
      float m_use, alpha;
      if constexpr (kMasked) {
        m_use = m_new == kNegInf ? 0.f : m_new;
        alpha = m_new == m_run[nb] ? 1.f : __builtin_amdgcn_exp2f(m_run[nb] - m_use);
      } else {
        m_use = m_new;  // finite
        alpha = m_new == m_run[nb] ? 1.f : __builtin_amdgcn_exp2f(m_run[nb] - m_new);
      }
      float pr[4];
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[i] = kMasked ? __builtin_amdgcn_exp2f(s[i] - m_use)
                        : __builtin_amdgcn_exp2f(__builtin_fmaf(acc[i], s2, -m_use));
        psum += pr[i];
      }
      l_run[nb] = l_run[nb] * alpha + psum;
      m_run[nb] = m_new;
      if (__ballot(alpha != 1.f) != 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = row_value<16>(alpha, g, i);
#pragma unroll
          for (int d = 0; d < 8; ++d) o[nb][d][i] *= a;
        }
      }
      pv_accumulate(o[nb], p_operand(pr), vb);
    }
  };

#if FK_PREFILL_PREFETCH
  // Register double buffer: the next tile's loads are issued before the current
  // tile is processed (the last tile re-reads itself, a cache hit).
  TileRegs<kFp8> cur;
  bool page_ok = false;
  if (ntiles > 0)
    prefill_load_tile<kFp8>(P, key_row<kPaged>(P, bt_row, k_start, 0, page_ok), row_cap, h, r, g,
                            cur);
  auto advance = [&](auto masked, int t) {
    const int tn = min(t + 1, ntiles - 1);
    bool ok_n;
    const int64_t row_n = key_row<kPaged>(P, bt_row, k_start, tn * kTile, ok_n);
    TileRegs<kFp8> nxt;
    prefill_load_tile<kFp8>(P, row_n, row_cap, h, r, g, nxt);
    tile_step(masked, t * kTile, cur, page_ok);
    cur = nxt;
    page_ok = ok_n;
  };
  int t = 0;
  if constexpr (kPaged) {
    // A masked page (-1 table entry) needs the mask, so full tiles are only
    // trusted while their pages are valid: check per tile.
    for (; t < nfull; ++t) {
      bool ok;
      (void)key_row<kPaged>(P, bt_row, k_start, t * kTile, ok);
      if (!ok) break;
      advance(std::false_type{}, t);
    }
  } else {
    for (; t < nfull; ++t) advance(std::false_type{}, t);
  }
  for (; t < ntiles; ++t) advance(std::true_type{}, t);
#else
  if constexpr (kChunk == 1) {
    // One tile at a time; the unmasked tiles (every query sees them in full)
    // come first, in their own loop, so each loop body holds one variant.  A
    // masked page (-1 table entry) needs the mask: the unmasked loop stops at
    // the first one (checked before its loads are issued).
    auto advance = [&](auto masked, int t) {
      bool ok;
      TileRegs<kFp8> cur;
      prefill_load_tile<kFp8>(P, key_row<kPaged>(P, bt_row, k_start, t * kTile, ok), row_cap, h,
                              r, g, cur);
      tile_step(masked, t * kTile, cur, ok);
    };
    int t = 0;
    for (; t < nfull; ++t) {
      if constexpr (kPaged) {
        bool ok;
        (void)key_row<kPaged>(P, bt_row, k_start, t * kTile, ok);
        if (!ok) break;
      }
      advance(std::false_type{}, t);
    }
    for (; t < ntiles; ++t) advance(std::true_type{}, t);
  } else {
  // Chunks of kChunk tiles: all their loads are issued, then the tiles are
  // processed in order (each waits only for its own loads).  A tile is
  // processed unmasked when every query sees it in full and its page is valid.
  for (int t0 = 0; t0 < ntiles; t0 += kChunk) {
    TileRegs<kFp8> buf[kChunk];
    bool ok[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      const int tt = min(t0 + u, ntiles - 1);
      prefill_load_tile<kFp8>(P, key_row<kPaged>(P, bt_row, k_start, tt * kTile, ok[u]), row_cap,
                              h, r, g, buf[u]);
    }
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      const int tt = t0 + u;
      if (tt >= ntiles) break;
      if (tt < nfull && ok[u])
        tile_step(std::false_type{}, tt * kTile, buf[u], true);
      else
        tile_step(std::true_type{}, tt * kTile, buf[u], ok[u]);
    }
  }
  }
#endif

  const float vs = (kFp8 && P.v_scale) ? P.v_scale[h] : 1.f;
#pragma unroll
  for (int nb = 0; nb < kColBlocks; ++nb) {
    const float l_col = pair_sum(l_run[nb]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int jr = j0 + 16 * nb + 4 * g + i;  // query row this lane holds
      const float l = row_value<16>(l_col, g, i);
      if (jr >= q_len) continue;
      const float f = l > 0.f ? vs / l : 0.f;
      uint32_t w[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const bf16x2_t pk = {static_cast<__bf16>(o[nb][2 * d][i] * f),
                             static_cast<__bf16>(o[nb][2 * d + 1][i] * f)};
        w[d] = __builtin_bit_cast(uint32_t, pk);
      }
      *reinterpret_cast<uint4*>(P.out + static_cast<int64_t>(q_start + jr) * P.out_row_stride +
                                static_cast<int64_t>(hq) * kHead + 8 * r) =
          make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

template <bool FP8, bool PAGED>
void launch_prefill(const PrefillParams& P, int nw, dim3 grid, const int32_t* bt,
                    const int32_t* cu_q, const int32_t* cu_k, hipStream_t stream) {
#define FK_PF(NW)                                                                        \
  hipLaunchKernelGGL((paged_prefill_kernel<NW, FP8, PAGED>), grid, dim3(NW * 64), 0, stream, \
                     P, bt, cu_q, cu_k)
  if (nw <= 1) FK_PF(1);
  else if (nw <= 2) FK_PF(2);
  else if (nw <= 4) FK_PF(4);
  else FK_PF(8);
#undef FK_PF
}

}  // namespace
}  // namespace fk

namespace fk {
namespace {

int prefill_entry(const char* name, bool paged, void* out, int64_t out_row_stride, const void* q,
                  int64_t q_row_stride, const void* k, int64_t k_row_bytes, const void* v,
                  int64_t v_row_bytes, int kv_dtype, const float* k_scale, const float* v_scale,
                  const int32_t* block_tables, int64_t bt_row_stride,
                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t batch,
                  int64_t max_seqlen_q, int num_heads, int num_kv_heads, int head_size,
                  int block_size, int64_t num_blocks, float scale, int causal, void* stream) {
  FK_REQUIRE(batch >= 0 && batch <= 65535, "%s: batch %lld out of range [0, 65535]", name,
             (long long)batch);
  FK_REQUIRE(max_seqlen_q >= 0 && max_seqlen_q <= (int64_t(1) << 30),
             "%s: max_seqlen_q %lld out of range", name, (long long)max_seqlen_q);
  FK_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             "%s: num_heads %d must be a positive multiple of num_kv_heads %d", name, num_heads,
             num_kv_heads);
  if (head_size != kHead)
    return set_error(FK_ERR_UNSUPPORTED, "%s: head_size %d unsupported (128 only)", name,
                     head_size);
  if (num_heads / num_kv_heads > 16)
    return set_error(FK_ERR_UNSUPPORTED, "%s: GQA group %d > 16 unsupported", name,
                     num_heads / num_kv_heads);
  FK_REQUIRE(num_kv_heads <= 32767, "%s: too many kv heads", name);
  if (paged) {
    FK_REQUIRE(block_size >= kTile && (block_size & (block_size - 1)) == 0,
               "%s: block_size %d must be a power of two >= 16", name, block_size);
    FK_REQUIRE(kv_dtype == FK_DTYPE_BF16 || kv_dtype == FK_DTYPE_FP8_E4M3FN,
               "%s: kv dtype %d unsupported (bf16 or fp8 e4m3fn)", name, kv_dtype);
  }
  FK_REQUIRE(q_row_stride >= static_cast<int64_t>(num_heads) * head_size &&
                 out_row_stride >= static_cast<int64_t>(num_heads) * head_size,
             "%s: row stride shorter than num_heads * head_size", name);
  const int64_t elem = kv_dtype == FK_DTYPE_FP8_E4M3FN ? 1 : 2;
  FK_REQUIRE(k_row_bytes >= num_kv_heads * kHead * elem && v_row_bytes >= num_kv_heads * kHead * elem,
             "%s: key/value rows shorter than num_kv_heads * head_size", name);
  if (batch == 0 || max_seqlen_q == 0) return FK_OK;
  FK_REQUIRE(out && q && k && v && cu_seqlens_q && cu_seqlens_k && (!paged || block_tables),
             "%s: null pointer", name);
  FK_REQUIRE(!paged || num_blocks >= 1, "%s: the cache must hold at least one block", name);
  FK_REQUIRE(aligned16(q) && aligned16(out) && aligned16(k) && aligned16(v) &&
                 q_row_stride % 8 == 0 && out_row_stride % 8 == 0 && k_row_bytes % 16 == 0 &&
                 v_row_bytes % 16 == 0,
             "%s: q/out/keys/values must be 16-byte aligned with 16-byte row strides", name);
  const int64_t qblocks = (max_seqlen_q + kQTokens - 1) / kQTokens;
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
  P.scale_log2 = scale * kLog2e;
  P.causal = causal ? 1 : 0;
  const int nw = P.gqa < 8 ? P.gqa : 8;  // waves (query heads) per work-group
  const int hsplit = (P.gqa + nw - 1) / nw;
  const dim3 grid(static_cast<unsigned>(qblocks), static_cast<unsigned>(num_kv_heads * hsplit),
                  static_cast<unsigned>(batch));
  hipStream_t s = as_stream(stream);
  if (!paged)
    launch_prefill<false, false>(P, nw, grid, nullptr, cu_seqlens_q, cu_seqlens_k, s);
  else if (kv_dtype == FK_DTYPE_FP8_E4M3FN)
    launch_prefill<true, true>(P, nw, grid, block_tables, cu_seqlens_q, cu_seqlens_k, s);
  else
    launch_prefill<false, true>(P, nw, grid, block_tables, cu_seqlens_q, cu_seqlens_k, s);
  return check_launch(name);
}

}  // namespace
}  // namespace fk

extern "C" int fk_paged_prefill(void* out, int64_t out_row_stride, const void* q,
                                int64_t q_row_stride, const void* k_cache, const void* v_cache,
                                int kv_dtype, const float* k_scale, const float* v_scale,
                                const int32_t* block_tables, int64_t bt_row_stride,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                int64_t batch, int64_t max_seqlen_q, int num_heads,
                                int num_kv_heads, int head_size, int block_size,
                                int64_t num_blocks, float scale, int causal, void* stream) {
  const int64_t row = static_cast<int64_t>(num_kv_heads) * head_size *
                      (kv_dtype == FK_DTYPE_FP8_E4M3FN ? 1 : 2);
  return fk::prefill_entry("fk_paged_prefill", true, out, out_row_stride, q, q_row_stride,
                           k_cache, row, v_cache, row, kv_dtype, k_scale, v_scale, block_tables,
                           bt_row_stride, cu_seqlens_q, cu_seqlens_k, batch, max_seqlen_q,
                           num_heads, num_kv_heads, head_size, block_size, num_blocks, scale,
                           causal, stream);
}

extern "C" int fk_varlen_prefill(void* out, int64_t out_row_stride, const void* q,
                                 int64_t q_row_stride, const void* key, int64_t key_row_stride,
                                 const void* value, int64_t value_row_stride,
                                 const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                 int64_t batch, int64_t max_seqlen_q, int num_heads,
                                 int num_kv_heads, int head_size, float scale, int causal,
                                 void* stream) {
  return fk::prefill_entry("fk_varlen_prefill", false, out, out_row_stride, q, q_row_stride, key,
                           key_row_stride * 2, value, value_row_stride * 2, FK_DTYPE_BF16,
                           nullptr, nullptr, nullptr, 0, cu_seqlens_q, cu_seqlens_k, batch,
                           max_seqlen_q, num_heads, num_kv_heads, head_size, 16, 0, scale, causal,
                           stream);
}
