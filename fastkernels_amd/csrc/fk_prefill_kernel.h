// Paged prefill attention kernel (variable-length query chunks over a paged KV
// cache, or over dense keys) for MI355X (gfx950).  The C entry points are in
// fk_paged_prefill.hip; fk_prefill_heads.hip instantiates the extra head sizes.
//
// Semantics: FlashAttnPrefill.forward with a block table
// (fastkernels/tasks/baseline/L1/flash_attn_prefill.py:28-74: flash_attn_varlen_func
// with cu_seqlens_q, seqused_k = cu_seqlens_k[1:] - cu_seqlens_k[:-1], causal), and
// the reference's torch fallback Attention._prefill_torch_from_cache
// (fastkernels/tasks/baseline/L2/attention_impl.py:640-652, _sdpa_one :606-622):
// sequence b owns query rows [cu_q[b], cu_q[b+1]) (q_len of them) and the first
// k_len = cu_k[b+1] - cu_k[b] tokens of its paged cache.  Query j (0-based in
// its chunk) sits at position k_len - q_len + j and sees keys
// [0, k_len - q_len + j] (causal, aligned to the end of the keys), or, under
// a sliding window (flash-attn window_size = (window_left, 0)), keys
// [k_len - q_len + j - window_left, k_len - q_len + j].  A query with no
// visible key gets a zero row.  Attention sinks (s_aux: one logit per query
// head) join each row's softmax denominator, as in the decode kernel.  kv head
// = hq / (Hq / Hk); fp8 pages are dequantised per kv head as in the decode
// kernel.  Optionally the kernel also writes each row's softmax log-sum-exp,
// lse = ln(sum_k e^(scale q.k)) (flash_attn_varlen_func's return_softmax_lse,
// fastkernels/tasks/baseline/L1/flash_attn_varlen.py:33-46; -inf for a row
// with no visible key), fp32 [Hq, total_q] with a row stride.
//
// Head sizes.  D (query / key) and DV (value) are template parameters, each a
// multiple of 8 up to 256 (fp8 pages: D = DV in {64, 128, 256}).  The score
// MFMAs run over D rounded up to 32 and P.V over DV rounded up to 16: the
// query's padding dims are zero and the key's are replaced by zeros in
// registers, so they add nothing; the value's padding dims only feed output
// dims that are never written.  In LDS a row is padded to a multiple of 64
// bytes (the padding is never loaded), so that 16 rows are whole 64-lane
// direct-to-LDS loads.  DV != D is MLA's prefill (query / key 192 = 128 nope +
// 64 rope, value 128; L2/mla_attention_impl.py:390-398).
//
// Work decomposition: work-group = 4 waves over one kv head and one block of
// query tokens of one sequence: the waves are the group's query heads (up to
// 4; larger groups span several work-groups) times consecutive 32-token query
// blocks (4 / heads of them).  A wave keeps two 16-query column blocks of one
// head in MFMA tiles (fk_attn_tile.h: S = K Q^T per 16-key tile, online
// softmax per query column, O += P V).  The work-group streams the keys in
// stages of 32 through LDS (double-buffered: the next stage's global loads are
// in flight while the current one is consumed), so the waves share each K/V
// byte and no wave waits on a global load per tile; each wave stops at its own
// last visible key.  In a causal chunk with few cached keys before it, a
// work-group takes two query blocks, one near the chunk's end and one near its
// start, so that the work-groups are even.
//
// Key split.  When the launch has too few work-groups to give every SIMD two
// waves (a single prompt: 2048 tokens over 8 kv heads make 256 work-groups
// after pairing), the work-group has 8 waves in two halves of 4: both halves
// take the same queries, the first half streams the first half of the block's
// key stages and the second half the rest, each through its own LDS buffers,
// in lock step (one barrier per stage; the half with fewer stages passes empty
// barriers).  At the end the second half leaves its (O, max, sum) in LDS and
// the first half merges them with the log-sum-exp rule before it writes the
// rows.  Each block's serial chain of stages halves, and every SIMD runs two
// waves.
#pragma once

#include <climits>
#include <type_traits>

#include "fk_attn_tile.h"

namespace fk {

struct PrefillParams {
  uint16_t* out;
  int64_t out_row_stride;
  const uint16_t* q;
  int64_t q_row_stride;
  const uint8_t* k_cache;  // paged: the caches; dense: the first key / value row
  const uint8_t* v_cache;
  int64_t k_row_bytes;     // bytes between key rows (paged: Hk * D * elem)
  int64_t v_row_bytes;     // bytes between value rows (paged: Hk * DV * elem)
  const float* k_scale;
  const float* v_scale;
  int64_t bt_row_stride;
  int num_kv_heads;
  int gqa;
  int block_size_log2;
  int64_t num_blocks;
  float scale_log2;
  int causal;        // 0: every query sees all k_len keys
  int window_left;   // causal sliding window: keys >= position - window_left (-1: none)
  const float* sinks;  // attention sink logits [num_heads] fp32, or nullptr
  float* lse;          // log-sum-exp [num_heads, lse_row_stride] fp32, or nullptr
  int64_t lse_row_stride;
  // Work-group key split: each query block's key stages are divided over xs
  // work-groups (1: none), which leave their partial states in `part` for
  // prefill_merge_kernel: O [xs][part_rows][num_heads][DV] bf16 (before the
  // division by the sum, rounded once), then from byte 2 xs part_rows num_heads
  // DV (a multiple of 16: DV is a multiple of 8) [xs][part_rows][num_heads][4]
  // fp32 (running max in log2 units, the sum the output divides by, the fp32 sum
  // of the log-sum-exp output, unused).
  int xs;
  void* part;
  int64_t part_rows;  // rows of q (at least cu_seqlens_q[batch])
  int num_heads;
};

// Floats of the partial state per (part, row, head) besides O.
constexpr int kPartMl = 4;
// The fp32 records of the key parts' states, after their bf16 O.
__host__ __device__ inline int64_t part_ml_offset(int xs, int64_t part_rows, int num_heads,
                                                  int dv) {
  return static_cast<int64_t>(xs) * part_rows * num_heads * dv * 2;
}
constexpr int kMaxKeyParts = 8;  // work-group key split: parts per query block at most

// Launches the kernel for the head sizes fk_prefill_heads.hip instantiates
// (besides D = DV in {64, 128, 256}); false when (D, DV) is not among them.
bool launch_prefill_extra(int D, int DV, bool paged, bool split, const PrefillParams& P,
                          dim3 grid, const int32_t* bt, const int32_t* cu_q,
                          const int32_t* cu_k, hipStream_t stream);

namespace {

#ifndef FK_PREFILL_COLS
#define FK_PREFILL_COLS 2
#endif
// Two waves per SIMD (two 4-wave work-groups per CU; each holds 32 KB of LDS for
// bf16 pages at head size 128, 64 KB at 256).  At 256 the bf16 P.V operands go
// in two halves to fit in the 256 registers two waves leave (fp8 fits as is);
// dense keys at 256 (the row clamping) would still spill 11 VGPRs, so one.
constexpr int prefill_waves_per_simd(int D, bool paged) { return D > 192 && !paged ? 1 : 2; }
#ifndef FK_PREFILL_LAZY
#define FK_PREFILL_LAZY 8.0f
#endif
constexpr int kColBlocks = FK_PREFILL_COLS;    // 16-query column blocks per wave
constexpr float kLazy = FK_PREFILL_LAZY;       // max-update threshold (log2 units)
#ifndef FK_PREFILL_FMA_EXP
#define FK_PREFILL_FMA_EXP 1
#endif
// The softmax's exponent argument s2 (K.Q) - m in one FMA per key (the lazy test
// on its lane max); 0: the scaled score, then the subtraction.
constexpr bool kFmaExp = FK_PREFILL_FMA_EXP;
constexpr float kFar = -1.0e30f;  // the max the exponent subtracts before a column's first key
constexpr int kQTokens = 16 * kColBlocks;      // query tokens per wave at head size 128
// Column blocks per wave at head sizes (D, DV): at 256 the O accumulators of one
// block (16 tiles of 4 fp32 per lane) already take what two take at 128; above
// 128 the query operands and key tiles of two blocks would not fit beside them.
constexpr int col_blocks_for(int D, int DV) { return (D > 128 || DV > 128) ? 1 : kColBlocks; }
// MFMA extents: the score MFMAs run over D rounded up to 32, P.V over DV rounded
// up to 16.
constexpr int qk_extent(int D) { return (D + 31) / 32 * 32; }
constexpr int v_extent(int DV) { return (DV + 15) / 16 * 16; }
constexpr int kPrefillWaves = 4;               // waves per work-group
#ifndef FK_PREFILL_STAGE
#define FK_PREFILL_STAGE 32
#endif

// bf16 V slices of a pair read right after its score MFMAs, so that their LDS
// latency passes under the softmax (1), or after the softmax (0).  Applies at
// value head sizes 128 .. 255 (below, the earlier reads measured slower).
#ifndef FK_PREFILL_VEARLY
#define FK_PREFILL_VEARLY 1
#endif

// Tile a's K chunks of an unmasked stage read right after the barrier, before
// the staging loads (1, head sizes 64 and 256), or with the pair's scores (0).
#ifndef FK_PREFILL_KEARLY
#define FK_PREFILL_KEARLY 1
#endif

// Causal pairs under the key split at heads of 128 and up: the second half streams
// the light block whole and the heavy block's tail (1), or both halves split both
// blocks (0).
#ifndef FK_PREFILL_SPLIT_PAIR
#define FK_PREFILL_SPLIT_PAIR 1
#endif
// Causal pairs in 4-wave work-groups: odd work-groups take their light block first
// (1), or every work-group its heavy block first (0).
#ifndef FK_PREFILL_ALT_ORDER
#define FK_PREFILL_ALT_ORDER 1
#endif

// fp8 pages: each stage converted once into bf16 LDS buffers (1), or every
// wave dequantising the K / V bytes it reads (0).
#ifndef FK_PREFILL_FP8_CONVERT
#define FK_PREFILL_FP8_CONVERT 1
#endif
// Keys per LDS stage (a multiple of 32).  Measured on MI355X (bf16, 1x2048,
// 4x512 over 4096, 16x512 prompts): 32 keys 102 / 220 / 89 us against 117 /
// 244 / 99 us for 64; again with the current loop, 88 / 187 / 83 against
// 98 / 208 / 91.
constexpr int kStageKeys = FK_PREFILL_STAGE;
constexpr int kStageTiles = kStageKeys / kTile;

__device__ __forceinline__ int64_t prefill_page(const PrefillParams& P,
                                                const int32_t* __restrict__ bt_row, int tok) {
  const int idx = tok >> P.block_size_log2;
  if (idx >= P.bt_row_stride) return -1;
  const int64_t page = bt_row[idx];
  return (page >= 0 && page < P.num_blocks) ? page : -1;
}

// The last block-table entry a wave looked up (wave-uniform), with the K and V
// rows of its page's first slot (the kv head's row of the caches): a page spans
// block_size / 32 stages, so most lookups reuse it instead of waiting for a
// scalar load, and a tile's source address is that row plus a 32-bit offset.
struct PageCache {
  int idx = -1;
  int64_t page = -1;             // the block-table entry (-1: masked; page 0 is read)
  const uint8_t* kb = nullptr;   // K row of the page's slot 0, kv head h
  const uint8_t* vb = nullptr;   // V row of the page's slot 0, kv head h
};

// Paged keys: the page of key `tok` into pc (a scalar load only when the page
// changes).
__device__ __forceinline__ void page_lookup(const PrefillParams& P,
                                            const int32_t* __restrict__ bt_row, int tok,
                                            const uint8_t* kh, const uint8_t* vh, PageCache& pc) {
  const int idx = tok >> P.block_size_log2;
  if (idx != pc.idx) {
    const int64_t page = prefill_page(P, bt_row, tok);
    const int64_t slot0 = (page < 0 ? 0 : page) << P.block_size_log2;
    pc.idx = idx;
    pc.page = page;
    pc.kb = kh + slot0 * P.k_row_bytes;
    pc.vb = vh + slot0 * P.v_row_bytes;
  }
}

// Whether key `tok` of the sequence is readable: paged, its page's block-table
// entry is not -1; dense keys always are.
template <bool kPaged>
__device__ __forceinline__ bool key_ok(const PrefillParams& P, const int32_t* __restrict__ bt_row,
                                       int tok, const uint8_t* kh, const uint8_t* vh,
                                       PageCache& pc) {
  if constexpr (kPaged) {
    page_lookup(P, bt_row, tok, kh, vh, pc);
    return pc.page >= 0;
  } else {
    return true;
  }
}

// LDS staging of key/value rows.  A stage is kStageKeys consecutive keys of one
// kv head: kStageKeys K rows, then kStageKeys V rows.  A row takes its 16-byte
// chunks padded to a multiple of 4 (the padding is never loaded), so that 16
// rows are whole 64-chunk loads; chunk q of row R is stored at chunk index
// q ^ (R mod M), M the largest power of two dividing the padded count, so that
// the row-parallel writes and the MFMA-layout reads (16 rows at one chunk
// index, or one row's 16 chunks) spread over the banks.
template <bool kFp8, int D, int DV>
struct Stage {
  static constexpr int kElt = kFp8 ? 1 : 2;
  static constexpr int kKReal = D * kElt / 16;  // chunks of a key row that hold data
  static constexpr int kVReal = DV * kElt / 16;
  static constexpr int kKChunks = (kKReal + 3) / 4 * 4;  // padded row lengths, in chunks
  static constexpr int kVChunks = (kVReal + 3) / 4 * 4;
  static constexpr int kKMask = (kKChunks & -kKChunks) - 1;
  static constexpr int kVMask = (kVChunks & -kVChunks) - 1;
  static constexpr int kNK = kStageKeys * kKChunks;  // chunk slots of the K rows
  static constexpr int kNV = kStageKeys * kVChunks;
  static constexpr int kBytes = 16 * (kNK + kNV);     // K rows + V rows
  // Direct-to-LDS loads per thread per stage (16 bytes each, 64 slots a load).
  static constexpr int kLoads = (kNK + kNV) / (kPrefillWaves * 64);
  static_assert(D * kElt % 16 == 0 && DV * kElt % 16 == 0, "rows of whole 16-byte chunks");
  static_assert((kNK + kNV) % (kPrefillWaves * 64) == 0, "whole loads per thread");
  __device__ __forceinline__ static int offset(int which, int row, int q) {
    return which == 0 ? (row * kKChunks + (q ^ (row & kKMask))) << 4
                      : (kNK + row * kVChunks + (q ^ (row & kVMask))) << 4;
  }
};

// 16 bytes from global memory straight into LDS (gfx950 global_load_lds_dwordx4):
// lane l of the wave writes at byte lds_addr + 16 l.  Written as inline asm, so
// the compiler's wait-count pass does not see it: its builtin form makes the
// pass wait for the load before every later LDS read, including reads of the
// other stage buffer, which would serialise the double buffer.  The kernel
// orders it explicitly instead (s_waitcnt vmcnt(0), then a barrier, before the
// buffer is read).  M0 carries the LDS address: an input operand bound to M0, so
// the compiler writes it (and knows it changed) with no save and restore; the
// s_nop is the wait state between that write and the load that reads M0.
__device__ __forceinline__ void lds_dma16(const uint8_t* src, uint32_t lds_addr) {
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(src), "{m0}"(lds_addr)
      : "memory");
}
// The same load with a wave-uniform 64-bit base in SGPRs and a per-lane 32-bit
// byte offset (the load's saddr form): lane l reads base + off.  A tile's base
// changes from stage to stage and the lanes' offsets do not, so a stage's
// loads take no 64-bit address arithmetic per lane.
__device__ __forceinline__ void lds_dma16_s(const uint8_t* base, uint32_t off, uint32_t lds_addr) {
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(off), "s"(base), "{m0}"(lds_addr)
      : "memory");
}

// Value of `x` held by lane 4g + i (g = this lane's row group, lanes 16g ..
// 16g + 15), for the O row 4g + i this lane accumulates: one cross-lane read
// (ds_bpermute) rather than four readlanes and a select chain, which the
// compiler turns into branches.
__device__ __forceinline__ float row_from(float x, int g, int i) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute((4 * g + i) * 4, __float_as_int(x)));
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr_of(const uint8_t* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t*)p));
}

// Floats one wave of the key split's second half leaves in LDS for its partner:
// O (kCB x D/16 MFMA tiles of 4 floats per lane), the row sums (kCB x 4 per
// lane) and the column maxima (kCB per lane).
template <int DVP, int kCB>
constexpr int split_exchange_floats() {
  return kCB * (DVP / 16) * 64 * 4 + kCB * 64 * 4 + kCB * 64;
}

// Tile tt (rows 16 tt .. 16 tt + 15) of a staged buffer in the register layout
// a global load of the tile would give (DTile, fk_attn_tile.h): the K rows (t.k)
// and, for fp8 stages, the V rows (t.v), read separately so that a caller can
// keep them apart in time.
template <bool kFp8, int D>
__device__ __forceinline__ void lds_tile_k(const uint8_t* buf, int tt, int r, int g,
                                           DTile<kFp8, D>& t) {
  using S = Stage<kFp8, D, D>;
  const int kr = 16 * tt + r;
  if constexpr (!kFp8) {
#pragma unroll
    for (int c = 0; c < D / 32; ++c)
      t.k[c] = *reinterpret_cast<const uint4*>(buf + S::offset(0, kr, 4 * c + g));
  } else {
#pragma unroll
    for (int c = 0; c < D / 64; ++c)
      t.k[c] = *reinterpret_cast<const uint4*>(buf + S::offset(0, kr, (D / 64) * g + c));
  }
}
// K operand chunks of tile tt of a bf16 stage: chunk c = dims 32c + 8g .. +7 of key
// row 16 tt + r, for c < qk_extent(D) / 32; chunks past the row's data are zero.
template <int D, int DV>
__device__ __forceinline__ void lds_k_chunks(const uint8_t* buf, int tt, int r, int g,
                                             uint4 (&kc)[qk_extent(D) / 32]) {
  using S = Stage<false, D, DV>;
  const int kr = 16 * tt + r;
#pragma unroll
  for (int c = 0; c < qk_extent(D) / 32; ++c) {
    const uint4 v = *reinterpret_cast<const uint4*>(buf + S::offset(0, kr, 4 * c + g));
    // (c is known after unrolling: only the chunk that crosses the row's end selects.)
    kc[c] = (4 * c + 3 < S::kKReal || 4 * c + g < S::kKReal) ? v : make_uint4(0, 0, 0, 0);
  }
}

// fp8 V rows 4g + i: lane r's D / 16 bytes (dims (D/16) r ..), inside one chunk.
template <bool kFp8, int D>
__device__ __forceinline__ void lds_tile_v(const uint8_t* buf, int tt, int r, int g,
                                           DTile<kFp8, D>& t) {
  static_assert(kFp8, "bf16 V rows are read with lds_v_slice");
  using S = Stage<kFp8, D, D>;
  const int byte = (D / 16) * r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    ld_words(buf + S::offset(1, 16 * tt + 4 * g + i, byte >> 4) + (byte & 15), t.v[i]);
}

// P.V operand of the 16-dim slice d of tile tt (bf16 stages), read with the LDS
// transpose load: lane (r, g) gets V[keys 16 tt + 4g .. 16 tt + 4g + 3][dim
// 16 d + r], the B-operand layout of the 16x16x16 MFMA, with no register
// regrouping.  ds_read_b64_tr_b16 gives lane j of each 16-lane group, as its
// element a, element j mod 4 of the 8 bytes addressed by lane 4a + j / 4; so
// lane 4a + q addresses row 4g + a, dims 16d + 4q .. 16d + 4q + 3.
template <int D, int DV>
__device__ __forceinline__ short4_t lds_v_slice(const uint8_t* buf, int tt, int d, int r, int g) {
  using S = Stage<false, D, DV>;
  const int row = 16 * tt + 4 * g + (r >> 2);
  const int q = r & 3;
  const int off = S::offset(1, row, 2 * d + (q >> 1)) + 8 * (q & 1);
  typedef __attribute__((address_space(3))) short4_t* lds_short4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4)(buf + off));
}
// Slice d of tiles tt and tt + 1 (va, vb).  At value head 64 (the swizzle repeats
// every 16 rows there) tile tt + 1's address is tile tt's plus a constant, which
// the read takes as its immediate offset: one address per slice instead of two.
// Same box, A/B in alternating processes, two rounds (us), with the ones operand
// kept in registers in both: Whisper heads 4x512 over 4096 118.7 / 119.0 ->
// 114.0 / 114.1; at value head 128 (also one address per slice) 4x512 over 4096
// 145.7 / 147.1 -> 149.2 / 152.6, so there each tile has its own addresses.
template <int D, int DV>
__device__ __forceinline__ void lds_v_slice2(const uint8_t* buf, int tt, int d, int r, int g,
                                             short4_t& va, short4_t& vb) {
  using S = Stage<false, D, DV>;
  if constexpr (S::kVMask < 16 && v_extent(DV) <= 64) {
    const int row = 16 * tt + 4 * g + (r >> 2);
    const int q = r & 3;
    const int off = S::offset(1, row, 2 * d + (q >> 1)) + 8 * (q & 1);
    typedef __attribute__((address_space(3))) short4_t* lds_short4;
    const uint8_t* p = buf + off;
    va = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4)p);
    vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4)(p + 16 * S::kVChunks * 16));
  } else {
    va = lds_v_slice<D, DV>(buf, tt, d, r, g);
    vb = lds_v_slice<D, DV>(buf, tt + 1, d, r, g);
  }
}

// Work-group = kPrefillWaves waves over one kv head: hw query heads of its group
// times qs = kPrefillWaves / hw blocks of kQTokens query tokens (a group larger
// than kPrefillWaves heads spans hsplit work-groups).  All waves share the K/V
// stages; each walks the tiles up to its own last visible key.
// kKS = 2: the key split (8 waves; head sizes up to 192, and 256 with paged keys).
// kLse: also write each row's log-sum-exp (P.lse).  The softmax denominator the
// output is divided by is summed from the same bf16 P weights as the numerator
// (an MFMA against ones); the log-sum-exp needs the exact sum, so it keeps an
// fp32 sum of P per query column besides (8 adds per column block and 32 keys).
template <bool kFp8, bool kPaged, int D, int DV, int kKS, bool kLse = false>
__global__ __launch_bounds__(kKS * kPrefillWaves * 64)
__attribute__((amdgpu_waves_per_eu(prefill_waves_per_simd(D > DV ? D : DV, kPaged)))) void
paged_prefill_kernel(PrefillParams P, const int32_t* __restrict__ block_tables,
                     const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k) {
  static_assert(!kFp8 || (D == DV && (D == 64 || D == 128 || D == 256)),
                "fp8 pages: equal query / value head sizes 64, 128 or 256");
  using S = Stage<kFp8, D, DV>;
  // fp8 pages: the work-group converts each staged stage once into a bf16
  // stage (float(x) * scale rounded to bf16, the value each wave would form),
  // and the waves compute on bf16 tiles, instead of each wave dequantising the
  // same K / V bytes for its own query head.  Up to head size 128 each fp8
  // buffer has its bf16 one (kConv); at 256 two of those would not fit in LDS
  // with two work-groups per CU, so one bf16 buffer serves the stages in turn
  // (kConv1: converted after every wave is done with the stage before, a second
  // barrier per stage).
  constexpr bool kConv = kFp8 && FK_PREFILL_FP8_CONVERT && D <= 128;
  constexpr bool kConv1 = kFp8 && FK_PREFILL_FP8_CONVERT && D > 128;
  constexpr bool kFp8T = kFp8 && !kConv && !kConv1;  // fp8 tiles in the compute path
  using SB = Stage<kFp8T, D, DV>;         // the layout the compute path reads
  static_assert(kKS == 1 || (kKS == 2 && (D <= 192 || kPaged)),
                "key split: two halves, head size <= 192 (256 with paged keys)");
  constexpr int kCB = col_blocks_for(D, DV);  // 16-query column blocks per wave
  constexpr int kQT = 16 * kCB;               // query tokens per wave
  constexpr int kDQ = qk_extent(D);           // score MFMA extent
  constexpr int kQC = kDQ / 32;               // score MFMAs per tile and column block
  constexpr int kDVP = v_extent(DV);          // P.V extent
  constexpr int kVS = kDVP / 16;              // P.V slices
  // Stage buffers (two or three per half; with kConv a bf16 buffer beside each
  // fp8 one), and with the key split the exchange area that reuses them once
  // the last stage is consumed.
  constexpr int kXFloats = split_exchange_floats<kDVP, kCB>() + (kLse ? kCB * 64 : 0);
  // Key split with one pair per stage: the halves run opposite phases (half 1
  // defers each pair's P.V past the next barrier), three stage buffers a half.
  // (At head size 256 three buffers a half would not fit in LDS, nor with the
  // fp8 stage conversion, whose bf16 buffers come beside the fp8 ones: two, in
  // phase.)
  constexpr bool kPingPong =
      kKS > 1 && kStageTiles == 2 && 6 * S::kBytes <= 120 * 1024 && !kConv && !kConv1;
  constexpr int kBufs = kPingPong ? 3 : 2;
  // Causal pairs under the key split: the halves take the blocks as described at
  // the block loop (FK_PREFILL_SPLIT_PAIR; bf16 stages, where no barrier precedes a
  // block's first step; query / key heads of 128 and up).  Same box, A/B in
  // alternating processes, two rounds, us: head 128 1x2048 61.2 / 60.9 -> 60.0 /
  // 59.6, 1x1024 37.9 / 37.9 -> 36.7 / 36.9; head 256 (Qwen3-Next heads) 1x2048
  // 67.4 / 67.4 -> 65.8 / 66.5; head 64 (Whisper heads) 1x2048 45.1 / 45.1 -> 46.7 /
  // 46.5, so not there.
  constexpr bool kSplitPair =
      FK_PREFILL_SPLIT_PAIR && kKS > 1 && !kConv && !kConv1 && kDQ >= 128;
  constexpr int kHalfBytes =  // a half's buffers
      kBufs * (S::kBytes + (kConv ? SB::kBytes : 0)) + (kConv1 ? SB::kBytes : 0);
  constexpr int kStageAll = kKS * kHalfBytes;
  constexpr int kXBytes = kKS > 1 ? kPrefillWaves * kXFloats * 4 : 0;
  __shared__ __align__(16) uint8_t lds_all[kStageAll > kXBytes ? kStageAll : kXBytes];
  // Grid: x = kv head (x hsplit), y = sequence, z = query block (x P.xs key
  // parts, the part fastest).  The block index varies slowest, so the
  // work-groups that have work (low z when blocks are paired) are dispatched
  // first and spread over every CU.
  const int b = blockIdx.y;
  const int hw = P.gqa < kPrefillWaves ? P.gqa : kPrefillWaves;  // heads per work-group
  const int qs = kPrefillWaves / hw;                             // query blocks per work-group
  const int hsplit = (P.gqa + hw - 1) / hw;
  const int h = blockIdx.x / hsplit;
  const int head0 = (blockIdx.x - h * hsplit) * hw;
  const int q_start = cu_q[b];
  const int q_len = cu_q[b + 1] - q_start;
  const int k_start = cu_k[b];
  const int k_len = cu_k[b + 1] - k_start;
  // Query blocks of the sequence at work-group granularity (wg_tokens queries
  // each).  When the causal triangle dominates the sequence's work (fewer than
  // q_len cached keys before the chunk), work-group p takes the pair of blocks
  // nqb - 1 - p (the most keys) and p (the fewest), one after the other, so its
  // work-groups stream about the same number of keys and no wave is left with a
  // long tail on its own; the upper half of the grid then has nothing to do.
  // Otherwise the blocks' key counts are close, and work-group x takes block
  // nqb - 1 - x alone (the heaviest first), keeping twice the work-groups.
  const int wg_tokens = qs * kQT;
  const int nqb = (q_len + wg_tokens - 1) / wg_tokens;
  const bool paired = P.causal && k_len - q_len < q_len;
  const int xs = P.xs;
  const int x = static_cast<int>(blockIdx.z) / xs;
  const int xpart = static_cast<int>(blockIdx.z) - x * xs;  // this work-group's key part
  if (x >= (paired ? (nqb + 1) / 2 : nqb)) return;  // uniform over the work-group
  const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = kKS > 1 ? wave_id / kPrefillWaves : 0;  // key-split half
  const int wave = wave_id & (kPrefillWaves - 1);           // role within the half
  uint8_t* const lds_half = lds_all + half * kHalfBytes;
  // Stage st's buffer: two alternate; with three, stage st mod 3.
  // buf_rot: added to the stage index when picking its buffer (a block that starts
  // right after another in the same half, split pairs below, takes the buffer the
  // previous block's next stage would have used).
  int buf_rot = 0;
  auto stage_buf = [&](int st) {
    return lds_half + (kBufs == 2 ? ((st + buf_rot) & 1) : (st + buf_rot) % kBufs) * S::kBytes;
  };
  // The LDS byte address of stage st's buffer, as an integer (M0 of the
  // direct-to-LDS loads; no generic-pointer conversion per stage).
  const uint32_t lds_half_addr = __builtin_amdgcn_readfirstlane(lds_addr_of(lds_half));
  auto stage_addr = [&](int st) -> uint32_t {
    return lds_half_addr +
           (kBufs == 2 ? ((st + buf_rot) & 1) : (st + buf_rot) % kBufs) * S::kBytes;
  };
  // The buffer the compute path reads stage st from: the staged one, or with
  // kConv its bf16 conversion.
  auto comp_buf = [&](int st) {
    if constexpr (kConv) return lds_half + kBufs * S::kBytes + (st & 1) * SB::kBytes;
    else if constexpr (kConv1) return lds_half + kBufs * S::kBytes;
    else return stage_buf(st);
  };
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int head = head0 + wave % hw;
  const int hq = h * P.gqa + (head < P.gqa ? head : 0);
  // Position of query 0; non-causal, every query sits past the last key.
  const int offset = P.causal ? k_len - q_len : k_len;
  const int32_t* bt_row = kPaged ? block_tables + static_cast<int64_t>(b) * P.bt_row_stride
                                 : nullptr;
  // Dense keys: rows past the sequence's last key would run off the tensor.
  const int64_t row_cap = kPaged ? INT64_MAX : static_cast<int64_t>(k_start) + max(k_len, 1) - 1;
  const float s2 = P.scale_log2;
  // fp8 dequant scales of kv head h (1 for bf16 pages or no scale tensor): each
  // K / V element enters the MFMAs as float(x) * scale rounded to bf16.
  const float ks = (kFp8 && P.k_scale) ? P.k_scale[h] : 1.f;
  const float vsc = (kFp8 && P.v_scale) ? P.v_scale[h] : 1.f;

  const int win = P.window_left;
  // Stages [st0, nstages) of 32 keys that query block qblk streams: up to its
  // last query's last key, from its first query's window start.
  auto block_stages = [&](int qblk, int& st0, int& nstages) {
    const int jw0 = qblk * wg_tokens;
    const int kend_wg = max(0, min(k_len, offset + min(jw0 + wg_tokens, q_len)));
    const int kbeg_wg = win >= 0 ? max(0, offset + jw0 - win) : 0;
    nstages = (kend_wg + kStageKeys - 1) / kStageKeys;
    st0 = min(kbeg_wg / kStageKeys, nstages);
  };

  // This work-group's stages [wlo, whi) of query block qblk (st0: the block's
  // first stage): all of them, or with the work-group key split part xpart of xs
  // equal parts (a part past the end is empty).
  auto wg_range = [&](int qblk, int& st0, int& wlo, int& whi) {
    int nstages;
    block_stages(qblk, st0, nstages);
    wlo = st0;
    whi = nstages;
    if (xs > 1) {
      const int n1 = (nstages - st0 + xs - 1) / xs;
      wlo = min(st0 + xpart * n1, nstages);
      whi = min(wlo + n1, nstages);
    }
  };
  // This half's stages [st_lo, st_hi) of block qblk and the barriers every wave
  // passes (nsteps): the work-group's range, or with the key split the first or
  // second half of it.  With the deferred P.V of the ping-pong the second half
  // ends about one stage after the first (head size 128, per-wave clock stamps:
  // 1.1 us), so the first half takes the extra stage of an even count and the
  // second half's tail runs under the first's last stage.
  auto stage_range = [&](int qblk, int& st0, int& st_lo, int& st_hi, int& nsteps) {
    int wlo, whi;
    wg_range(qblk, st0, wlo, whi);
    st_lo = wlo;
    st_hi = whi;
    nsteps = whi - wlo;
    if constexpr (kKS > 1) {
      const int m = whi - wlo;
      // the first half's stages (at head size 64 the second half measured no lag)
      const int h0 = (kPingPong && kDQ > 64) ? min(m, (m + 2) / 2) : (m + 1) / 2;
      st_lo = half == 0 ? wlo : wlo + h0;
      st_hi = half == 0 ? wlo + h0 : whi;
      nsteps = h0;
    }
  };

  PageCache pc;
  // One query block of the work-group, start to finish: this half streams stages
  // [st_lo, st_hi) of it (st0: the block's first stage) and every wave passes
  // nsteps step barriers; with the key split the halves then merge (unless solo:
  // a block this half streams whole, which writes its own rows).
  auto process_block = [&](int qblk, int st0, int st_lo, int st_hi, int nsteps, bool solo) {
  const int jw0 = qblk * wg_tokens;  // first query of the work-group
  const int j0 = jw0 + (wave / hw) * kQT;
  // Waves without queries (past the chunk, or past the group) still stage.
  const bool active = j0 < q_len && head < P.gqa && wave < qs * hw;
  // Keys [0, kend) cover every query of this wave's block.
  const int kend = active ? max(0, min(k_len, offset + min(j0 + kQT, q_len))) : 0;
  // Sliding window: query j sees keys from offset + j - win.  kbeg (this wave's
  // first query) bounds the keys from below; the work-group starts streaming at
  // the stage holding its first query's (block_stages), and a stage at or after
  // khead (the last query's window start) is inside every query's window.
  const int kbeg = (win >= 0 && active) ? max(0, offset + j0 - win) : 0;
  const int khead = (win >= 0 && active) ? offset + min(j0 + kQT, q_len) - 1 - win : 0;

  // Q^T operands: column r of block nb = query j0 + 16 nb + r (dims past D zero).
  bf16x8_t qb[kCB][kQC];
#pragma unroll
  for (int nb = 0; nb < kCB; ++nb) {
    const int j = j0 + 16 * nb + r;
    const bool ok = active && j < q_len;
    const uint16_t* qp = P.q + static_cast<int64_t>(q_start + (ok ? j : 0)) * P.q_row_stride +
                         static_cast<int64_t>(hq) * D;
#pragma unroll
    for (int c = 0; c < kQC; ++c) {
      const int d0 = kFp8T ? (D / 4) * g + 8 * c : 32 * c + 8 * g;
      const uint4 v = (ok && d0 < D) ? *reinterpret_cast<const uint4*>(qp + d0)
                                     : make_uint4(0, 0, 0, 0);
      qb[nb][c] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  // Running max per query column (log2 units, this lane's column r), and the
  // softmax denominators in the O layout: l_acc[nb][i] is the sum for query row
  // 4g + i, accumulated by an MFMA of P against ones beside the P.V ones (the
  // same bf16 P weights as the numerator), so no VALU adds and no cross-lane
  // fetch at the end.
  float m_run[kCB];
  // kFmaExp: the max the exponent subtracts, m_run once it is finite and kFar
  // before (so that the first visible score of a column exceeds it by more than
  // kLazy and takes the rescale branch, which sets m_run).
  float m_ref[kCB];
  floatx4_t o[kCB][kVS], l_acc[kCB];
  // kLse: this lane's fp32 share of its query column's sum (keys 4g .. 4g + 3 of
  // every tile), against m_run.
  float l32[kCB];
#pragma unroll
  for (int nb = 0; nb < kCB; ++nb) {
    m_run[nb] = kNegInf;
    m_ref[nb] = kFar;
    l32[nb] = 0.f;
    l_acc[nb] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < kVS; ++d) o[nb][d] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  }
  // (Passed through an empty asm so that it stays in four VGPRs: as a constant the
  // compiler rebuilt it with five moves in every stage.  Same box, A/B in
  // alternating processes, two rounds, us: 4x512 over 4096 148.4 / 151.2 ->
  // 145.7 / 147.1, Qwen3-Next heads 1x2048 68.4 / 68.7 -> 67.4 / 67.5.)
  uint4 ones_w = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
  asm volatile("" : "+v"(ones_w.x), "+v"(ones_w.y), "+v"(ones_w.z), "+v"(ones_w.w));
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, ones_w);

  const int ntiles = (kend + kTile - 1) / kTile;
  // Tiles every query of the block sees in full need no mask: keys up to
  // offset + j0 (query j0's last key), inside [0, kend).
  const int nfull = active ? max(0, min(kend, offset + j0 + 1)) / kTile : 0;
  const int tbeg = kbeg / kTile;  // this wave's first tile

  // Two 16-key tiles (tiles tt, tt + 1 of `buf`, keys tok0 .. tok0 + 31):
  // scores, one online-softmax update per query column for the 32 keys, P.V.
  // kMasked applies the causal / length / window / page mask; unmasked pairs skip
  // it (every score is finite there, so the running max never stays -inf).
  // Updating the running max, the rescale test and the cross-lane row max once
  // per 32 keys instead of per 16 halves that part of the VALU work, and the two
  // tiles' score MFMAs form independent chains.  The V rows are read only after
  // the scores of both column blocks are done, so K, the scores and V are never
  // all live at once.
  //
  // pair_scores runs the scores and the softmax update (P into p_a / p_b) and
  // returns whether the pair's V rows need masking; pair_pv runs P.V.
  // Same box, A/B in alternating processes, two rounds (µs): 1x2048 60.3 / 59.6 ->
  // 59.6 / 59.0, 4x512 over 4096 161.9 / 160.2 -> 155.9 / 156.3, 16x512 75.6 / 76.1 ->
  // 74.2 / 74.5; at head size 64 (Whisper heads, 4x512 over 4096) 124.9 -> 128.1.
  constexpr bool kVEarly = FK_PREFILL_VEARLY && !kFp8T && kDVP >= 128 && kDVP < 256;
  short4_t vpre_a[kVS], vpre_b[kVS];  // kVEarly: the pair's V slices, read with its scores
  // kKEarly: tile a's K chunks of an unmasked stage, read right after the barrier,
  // before the stage's staging loads are issued, so that the scalar work of the
  // staging covers their LDS latency.  Same box, A/B in alternating processes, two
  // rounds (us): head 64 (Whisper heads) 4x512 over 4096 127.9 / 128.2 -> 121.2 /
  // 120.6, 1x2048 48.8 / 48.9 -> 47.7 / 47.4; head 256 (Qwen3-Next heads) 1x2048
  // 70.1 / 70.0 -> 68.7 / 68.4; at head 128 level to 1% slower (16x512 73.2 / 72.5
  // -> 74.0 / 73.0), so not there, nor at the sizes not measured.
  constexpr bool kKEarly =
      FK_PREFILL_KEARLY && !kFp8T && kStageTiles == 2 && (kDQ == 64 || kDQ == 256);
  uint4 kpre[kQC];
  bool kpre_ok = false;  // wave-uniform: kpre holds this pair's tile a
  auto pair_scores = [&](auto masked, int tok0, const uint8_t* buf, int tt, bool ok_a,
                         bool ok_b, short4_t (&p_a)[kCB], short4_t (&p_b)[kCB],
                         auto early) __attribute__((always_inline)) {
    constexpr bool kMasked = decltype(masked)::value;
    DTile<kFp8T, D> ta, tb;
    // Scores of tile a for every column block, then tile b's K is read: the two
    // K tiles are never live at once (20 fewer VGPRs in the compiler's own
    // allocation; measured 1% faster).
    floatx4_t sc_a[kCB], sc_b[kCB];
    // The MFMA blocks run at raised wave priority: while one wave of a SIMD is in
    // its softmax, the other's MFMAs issue first (4x512 chunks over 4096 keys
    // 174.3 -> 168.7 us; the shorter cases unchanged).
    __builtin_amdgcn_s_setprio(1);
    {
      uint4 ka[kQC];
      if constexpr (kFp8T) {
        lds_tile_k<kFp8T, D>(buf, tt, r, g, ta);
        k_chunks_d(ta, ka, ks);
      } else {
        if (kKEarly && kpre_ok) {
#pragma unroll
          for (int c = 0; c < kQC; ++c) ka[c] = kpre[c];
        } else {
          lds_k_chunks<D, DV>(buf, tt, r, g, ka);
        }
      }
#pragma unroll
      for (int nb = 0; nb < kCB; ++nb) sc_a[nb] = qk_scores_n(ka, qb[nb]);
    }
    asm volatile("" ::: "memory");  // tile b's K reads stay after tile a's
    {
      uint4 kb[kQC];
      if constexpr (kFp8T) {
        lds_tile_k<kFp8T, D>(buf, tt + 1, r, g, tb);
        k_chunks_d(tb, kb, ks);
      } else {
        lds_k_chunks<D, DV>(buf, tt + 1, r, g, kb);
      }
#pragma unroll
      for (int nb = 0; nb < kCB; ++nb) sc_b[nb] = qk_scores_n(kb, qb[nb]);
    }
    if constexpr (kVEarly && decltype(early)::value) {
      asm volatile("" ::: "memory");  // after tile b's K reads
#pragma unroll
      for (int d = 0; d < kVS; ++d) {
        lds_v_slice2<D, DV>(buf, tt, d, r, g, vpre_a[d], vpre_b[d]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int nb = 0; nb < kCB; ++nb) {
      const floatx4_t acc_a = sc_a[nb];
      const floatx4_t acc_b = sc_b[nb];
      const int j = j0 + 16 * nb + r;  // this lane's query column
      const int last = offset + j;     // its last visible key
      // Masked pairs: key tok0 + rel (rel = 16 * tile + 4g + e) is visible when
      // its tile's page is readable and dl <= rel - 4g <= dh: one range test per
      // key instead of the causal, length, chunk and window tests each.
      // Scores in log2 units, s2 * (K.Q), formed by an FMA or a product: either
      // result is canonical, so the max below compiles to plain v_max3 with no
      // NaN-quieting step per operand (as the raw MFMA results would need).
      // Masked keys take -inf in the max and P = 0 after the exponent.
      float s[8], sm[8];
      bool ok[8];
      int dh = 0, dl = 0;
      if constexpr (kMasked) {
        const int hi = j < q_len ? min(last, kend - 1) : -1;  // last visible key
        const int lo = win >= 0 ? last - win : 0;             // first visible key
        dh = hi - tok0 - 4 * g;
        dl = lo - tok0 - 4 * g;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (kMasked) {
          const int rel = (i >> 2) * kTile + (i & 3);  // compile-time
          ok[i] = ((i >> 2) ? ok_b : ok_a) && rel <= dh && rel >= dl;
        } else {
          ok[i] = true;
        }
      }
      float pr[8];
      if constexpr (kFmaExp) {
        // The exponent's argument in one FMA per key, s2 (K.Q) - m_ref, whose
        // lane max is the lazy test (an FMA result is canonical: plain v_max3).
        // The scaled score itself is formed only in the rare rescale branch.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s[i] = __builtin_fmaf(acc_a[i], s2, -m_ref[nb]);
          s[4 + i] = __builtin_fmaf(acc_b[i], s2, -m_ref[nb]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) sm[i] = ok[i] ? s[i] : kNegInf;
        const float lt = fmaxf(fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3])),
                               fmaxf(fmaxf(sm[4], sm[5]), fmaxf(sm[6], sm[7])));
        if (__ballot(lt > kLazy) != 0) {
          // A visible key's argument is finite, a masked one's -inf: the masks
          // need not stay live through the loop body.
          auto acc_of = [&](int i) { return i < 4 ? acc_a[i] : acc_b[i - 4]; };
          float ls = kNegInf;  // this lane's max of the scaled visible scores
#pragma unroll
          for (int i = 0; i < 8; ++i)
            ls = fmaxf(ls, (kMasked && sm[i] == kNegInf) ? kNegInf : acc_of(i) * s2);
          const float mt = pair_max(ls);
          const float m_new = mt > m_run[nb] + kLazy ? mt : m_run[nb];
          const float alpha = m_new == m_run[nb] ? 1.f : __builtin_amdgcn_exp2f(m_run[nb] - m_new);
          m_run[nb] = m_new;
          m_ref[nb] = m_new == kNegInf ? kFar : m_new;
          if constexpr (kLse) l32[nb] *= alpha;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float a = row_from(alpha, g, i);
#pragma unroll
            for (int d = 0; d < kVS; ++d) o[nb][d][i] *= a;
            l_acc[nb][i] *= a;
          }
#pragma unroll
          for (int i = 0; i < 8; ++i)
            sm[i] = (kMasked && sm[i] == kNegInf) ? kNegInf
                                                  : __builtin_fmaf(acc_of(i), s2, -m_ref[nb]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) pr[i] = __builtin_amdgcn_exp2f(sm[i]);
      } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[i] = acc_a[i] * s2;
        s[4 + i] = acc_b[i] * s2;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) sm[i] = ok[i] ? s[i] : kNegInf;
      // This lane's max over its 8 keys of the column.
      const float lt = fmaxf(fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3])),
                             fmaxf(fmaxf(sm[4], sm[5]), fmaxf(sm[6], sm[7])));
      // Lazy rescaling: the running max only moves when a score exceeds it by
      // more than kLazy (log2 units), so P <= 2^kLazy and the O / l rescale (a
      // cross-lane fetch per row) is rare after the first tiles.  The test
      // needs no cross-lane max: some column's max exceeds its m_run + kLazy
      // exactly when some lane's own max does, and the ballot spans every
      // lane.  The column max itself is taken only in the rare branch.  The
      // final normalisation divides by l accumulated against the same max, so
      // the result is unchanged up to rounding.
      if (__ballot(lt > m_run[nb] + kLazy) != 0) {
        const float mt = pair_max(lt);
        const float m_new = mt > m_run[nb] + kLazy ? mt : m_run[nb];
        // 1 where the column's max stays (also -inf to -inf), 0 from -inf.
        const float alpha = m_new == m_run[nb] ? 1.f : __builtin_amdgcn_exp2f(m_run[nb] - m_new);
        m_run[nb] = m_new;
        if constexpr (kLse) l32[nb] *= alpha;  // column layout, like alpha
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = row_from(alpha, g, i);
#pragma unroll
          for (int d = 0; d < kVS; ++d) o[nb][d][i] *= a;
          l_acc[nb][i] *= a;
        }
      }
      // A column with no visible key yet (masked stages only) keeps m = -inf;
      // all its P are masked to 0.
      const float m_use = (kMasked && m_run[nb] == kNegInf) ? 0.f : m_run[nb];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        // Masked scores are -inf in sm, so their P is 2^-inf = 0.
        pr[i] = __builtin_amdgcn_exp2f(sm[i] - m_use);
      }
      }
      const float (&pa)[4] = *reinterpret_cast<const float(*)[4]>(&pr[0]);
      const float (&pb)[4] = *reinterpret_cast<const float(*)[4]>(&pr[4]);
      p_a[nb] = p_operand(pa);
      p_b[nb] = p_operand(pb);
      if constexpr (kLse)
        l32[nb] += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
    }
    // Keys past the wave's keys (or on a masked page) may hold anything in V.
    // A pair of readable tiles wholly below kend (the causal diagonal of a
    // prompt) needs no V mask.
    return kMasked && (!ok_a || !ok_b || tok0 + 2 * kTile > kend);
  };
  auto pair_pv = [&](int tok0, const uint8_t* buf, int tt, bool ok_a, bool ok_b, bool vmask,
                     const short4_t (&p_a)[kCB], const short4_t (&p_b)[kCB],
                     auto early) __attribute__((always_inline)) {
    asm volatile("" ::: "memory");  // V reads stay after the score work
    if constexpr (!kFp8T && kDVP >= 256) {
      // bf16 at head size 256: the V slices go in two halves (read, mask, MFMAs),
      // so that half the V operands are live at once and two waves fit on a
      // SIMD; otherwise as below.
      constexpr int kDS = kVS / 2;  // slices per half
      uint32_t ma[2] = {~0u, ~0u}, mb[2] = {~0u, ~0u};
      if (vmask) {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const int k0 = tok0 + 4 * g + 2 * h2;
          ma[h2] = ((ok_a && k0 < kend) ? 0x0000ffffu : 0u) | ((ok_a && k0 + 1 < kend) ? 0xffff0000u : 0u);
          mb[h2] = ((ok_b && k0 + kTile < kend) ? 0x0000ffffu : 0u) |
                   ((ok_b && k0 + kTile + 1 < kend) ? 0xffff0000u : 0u);
        }
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        if (hh > 0) asm volatile("" ::: "memory");  // the second half's reads after the first's MFMAs
        short4_t vba[kDS], vbb[kDS];
#pragma unroll
        for (int d = 0; d < kDS; ++d) {
          lds_v_slice2<D, DV>(buf, tt, hh * kDS + d, r, g, vba[d], vbb[d]);
        }
        if (vmask) {
#pragma unroll
          for (int d = 0; d < kDS; ++d) {
            uint2 wa = __builtin_bit_cast(uint2, vba[d]), wb = __builtin_bit_cast(uint2, vbb[d]);
            wa.x &= ma[0]; wa.y &= ma[1];
            wb.x &= mb[0]; wb.y &= mb[1];
            vba[d] = __builtin_bit_cast(short4_t, wa);
            vbb[d] = __builtin_bit_cast(short4_t, wb);
          }
        }
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int nb = 0; nb < kCB; ++nb) {
          const bf16x8_t pab = __builtin_bit_cast(
              bf16x8_t, make_uint4(__builtin_bit_cast(uint2, p_a[nb]).x,
                                   __builtin_bit_cast(uint2, p_a[nb]).y,
                                   __builtin_bit_cast(uint2, p_b[nb]).x,
                                   __builtin_bit_cast(uint2, p_b[nb]).y));
#pragma unroll
          for (int d = 0; d < kDS; ++d) {
            const uint2 va = __builtin_bit_cast(uint2, vba[d]), vb = __builtin_bit_cast(uint2, vbb[d]);
            const bf16x8_t v8 = __builtin_bit_cast(bf16x8_t, make_uint4(va.x, va.y, vb.x, vb.y));
            o[nb][hh * kDS + d] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(pab, v8, o[nb][hh * kDS + d], 0, 0, 0);
          }
          if (hh == 1)
            l_acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pab, ones, l_acc[nb], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
      }
      return;
    }
    short4_t vba[kVS], vbb[kVS];  // shared by the column blocks
    if constexpr (!kFp8T) {
      // Slice d holds dims 16d .. 16d + 15 (lane r: dim 16d + r).
#pragma unroll
      for (int d = 0; d < kVS; ++d) {
        if constexpr (kVEarly && decltype(early)::value) {
          vba[d] = vpre_a[d];
          vbb[d] = vpre_b[d];
        } else {
          lds_v_slice2<D, DV>(buf, tt, d, r, g, vba[d], vbb[d]);
        }
      }
      // Zero the masked keys' V rows so that P = 0 never meets a NaN.
      if (vmask) {
        uint32_t ma[2], mb[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const int k0 = tok0 + 4 * g + 2 * h2;
          ma[h2] = ((ok_a && k0 < kend) ? 0x0000ffffu : 0u) | ((ok_a && k0 + 1 < kend) ? 0xffff0000u : 0u);
          mb[h2] = ((ok_b && k0 + kTile < kend) ? 0x0000ffffu : 0u) |
                   ((ok_b && k0 + kTile + 1 < kend) ? 0xffff0000u : 0u);
        }
#pragma unroll
        for (int d = 0; d < kVS; ++d) {
          uint2 wa = __builtin_bit_cast(uint2, vba[d]), wb = __builtin_bit_cast(uint2, vbb[d]);
          wa.x &= ma[0]; wa.y &= ma[1];
          wb.x &= mb[0]; wb.y &= mb[1];
          vba[d] = __builtin_bit_cast(short4_t, wa);
          vbb[d] = __builtin_bit_cast(short4_t, wb);
        }
      }
    } else {
      // Slice d holds dims (D/16) r + d (lane r), packed from the row loads.
      DTile<kFp8T, D> ta, tb;
      lds_tile_v<kFp8T, D>(buf, tt, r, g, ta);
      lds_tile_v<kFp8T, D>(buf, tt + 1, r, g, tb);
      bool keep_a[4], keep_b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        keep_a[i] = ok_a && tok0 + 4 * g + i < kend;
        keep_b[i] = ok_b && tok0 + kTile + 4 * g + i < kend;
      }
      const bool vall = !vmask;
      v_operands_fp8(ta, vsc, vall, keep_a, vba);
      v_operands_fp8(tb, vsc, vall, keep_b, vbb);
    }
    __builtin_amdgcn_s_setprio(1);
    // P.V over the 32 keys with the 16x16x32 MFMA (the 16x16x16 one takes as
    // long on gfx950 for half the work).  Its k index 8g + e stands for key
    // 4g + e of tile a (e < 4) and 4g + e - 4 of tile b (e >= 4): the A operand
    // (P) and the B operand (V) both take tile a's four keys then tile b's, so
    // the sum runs over the same 32 keys.
#pragma unroll
    for (int nb = 0; nb < kCB; ++nb) {
      const bf16x8_t pab = __builtin_bit_cast(
          bf16x8_t, make_uint4(__builtin_bit_cast(uint2, p_a[nb]).x,
                               __builtin_bit_cast(uint2, p_a[nb]).y,
                               __builtin_bit_cast(uint2, p_b[nb]).x,
                               __builtin_bit_cast(uint2, p_b[nb]).y));
#pragma unroll
      for (int d = 0; d < kVS; ++d) {
        const uint2 va = __builtin_bit_cast(uint2, vba[d]), vb = __builtin_bit_cast(uint2, vbb[d]);
        const bf16x8_t v8 = __builtin_bit_cast(bf16x8_t, make_uint4(va.x, va.y, vb.x, vb.y));
        o[nb][d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pab, v8, o[nb][d], 0, 0, 0);
      }
      l_acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pab, ones, l_acc[nb], 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // Staging with direct global-to-LDS loads (lds_dma16).  Load i of wave w
  // fills the stage's chunk slots p = 64 (4 i + w) + lane (the K rows' slots,
  // then the V rows'); slot p is physical chunk p mod C of row p / C (C the
  // padded row length), so the lane reads the logical chunk that the swizzle
  // puts there, or nothing when that chunk is row padding.  Rows of a masked
  // page (-1 table entry) read page 0 and rows past a dense tensor's end re-read
  // its last row; the consumer masks both.
  // All lanes of load i fall in one tile of the stage, of K or of V (a load
  // covers 64 slots, 16 rows are a multiple of 64 slots, and the slots are
  // 64-aligned), so its source address is a wave-uniform part (that tile's
  // first row) plus a per-lane part that does not change from stage to stage,
  // computed once here.
  constexpr int64_t kElt = kFp8 ? 1 : 2;
  const int64_t k_head_off = static_cast<int64_t>(h) * D * kElt;
  const int64_t v_head_off = static_cast<int64_t>(h) * DV * kElt;
  // Row 0 of the caches (paged) or of the tensors (dense) at kv head h.
  const uint8_t* const kh = P.k_cache + k_head_off;
  const uint8_t* const vh = P.v_cache + v_head_off;
  // Slot -> (K or V, row, logical chunk) of load i for this lane.
  auto slot_of = [&](int i, int& which, int& row, int& q) {
    const int pos = 64 * (kPrefillWaves * i + wave) + lane;
    which = pos >= S::kNK;
    const int rel = pos - (which ? S::kNK : 0);
    if (which) {
      row = rel / S::kVChunks;
      q = (rel - row * S::kVChunks) ^ (row & S::kVMask);
    } else {
      row = rel / S::kKChunks;
      q = (rel - row * S::kKChunks) ^ (row & S::kKMask);
    }
  };
  // The lane's byte offset from its tile's first row, for load i.
  uint32_t lane_off[S::kLoads];
  // Whether the lane's slot of load i holds data (not row padding).
  bool lane_ld[S::kLoads];
#pragma unroll
  for (int i = 0; i < S::kLoads; ++i) {
    int which, row, q;
    slot_of(i, which, row, q);
    const int64_t rb = which ? P.v_row_bytes : P.k_row_bytes;
    lane_off[i] = static_cast<uint32_t>((row & 15) * rb + 16 * q);
    lane_ld[i] = q < (which ? S::kVReal : S::kKReal);
  }
  // The first stage staged with a masked page (a -1 block-table entry), or
  // INT_MAX: the unmasked loop stops before it, so that it needs no page lookups
  // of its own.  Stages are staged in increasing order and before they are
  // consumed, so every stage below it that has been staged is readable.
  int ok_until = INT_MAX;
  const uint32_t slot_mask = (1u << P.block_size_log2) - 1;
  auto stage_load = [&](int st) {
    const uint32_t buf_addr = stage_addr(st);  // wave-uniform (the buffer is the half's)
    // First K and V rows of the stage's tiles, wave-uniform: paged, the cached
    // page's slot-0 rows plus the slot's 32-bit offset in the page (the host
    // bounds a page's bytes below 2^32); dense, row k_start + token.
    const uint8_t* kt[kStageTiles];
    const uint8_t* vt[kStageTiles];
    int64_t row0[kStageTiles];  // dense keys: the tiles' first rows
    bool all_ok = true;
#pragma unroll
    for (int tt = 0; tt < kStageTiles; ++tt) {
      const int tok = st * kStageKeys + tt * kTile;
      if constexpr (kPaged) {
        page_lookup(P, bt_row, tok, kh, vh, pc);  // the cached page unless it changes
        all_ok = all_ok && pc.page >= 0;
        const uint32_t slot = static_cast<uint32_t>(tok) & slot_mask;
        kt[tt] = pc.kb + slot * static_cast<uint32_t>(P.k_row_bytes);
        vt[tt] = pc.vb + slot * static_cast<uint32_t>(P.v_row_bytes);
        row0[tt] = 0;
      } else {
        row0[tt] = static_cast<int64_t>(k_start) + tok;
        kt[tt] = kh + row0[tt] * P.k_row_bytes;
        vt[tt] = vh + row0[tt] * P.v_row_bytes;
      }
    }
    if (!all_ok) ok_until = min(ok_until, st);
#pragma unroll
    for (int i = 0; i < S::kLoads; ++i) {
      const int pos0 = 64 * (kPrefillWaves * i + wave);  // wave-uniform
      const int which = pos0 >= S::kNK;                   // 0: K, 1: V
      const int tt = which ? ((pos0 - S::kNK) / S::kVChunks) >> 4 : (pos0 / S::kKChunks) >> 4;
      const uint8_t* base = which ? vt[0] : kt[0];
      int64_t first = row0[0];
#pragma unroll
      for (int u = 1; u < kStageTiles; ++u)
        if (tt == u) {
          base = which ? vt[u] : kt[u];
          first = row0[u];
        }
      if (kPaged || first + 15 <= row_cap) {
        // (padded rows: the padding chunks are not loaded)
        if ((S::kKReal == S::kKChunks && S::kVReal == S::kVChunks) || lane_ld[i])
          lds_dma16_s(base, lane_off[i], buf_addr + 16 * pos0);
      } else {
        // Dense keys whose tile runs past the tensor's end: clamp each row.
        int wh, row, q;
        slot_of(i, wh, row, q);
        const int64_t rb = which ? P.v_row_bytes : P.k_row_bytes;
        const uint8_t* src = (which ? vh : kh) + min(first + (row & 15), row_cap) * rb + 16 * q;
        if (lane_ld[i]) lds_dma16(src, buf_addr + 16 * pos0);
      }
    }
  };
  // Key split, half 1: each pair's P.V waits for the next step and runs right
  // after its barrier, before that step's loads and scores (the pair's V stays in
  // its stage buffer: three buffers per half, so the loads issued in step s,
  // into buffer (s + 1) mod 3, never meet the V of stage s - 1).  The two halves
  // then run opposite phases between barriers: while half 0's waves issue
  // their score MFMAs half 1's run the previous softmax's P.V, and while half 0
  // runs its softmax half 1 issues score MFMAs, instead of both waves of a SIMD
  // contending for the same pipe at the same time.
  short4_t pend_pa[kCB], pend_pb[kCB];  // P of the pending pair
  bool pend = false, pend_ok_a = true, pend_ok_b = true, pend_vm = false;
  int pend_tok0 = 0;
  const uint8_t* pend_buf = nullptr;
  // Consumes one stage from `buf` (this wave's tiles only, two at a time; a pair
  // whose second tile is past the wave's keys has those keys masked), every pair
  // with the mask or every pair without it: one variant per loop body keeps the
  // register count where two waves fit on a SIMD.  With `defer` (half 1 of the
  // key split, one pair per stage) the pair's P.V is left pending.
  auto stage_compute = [&](auto masked, int st, const uint8_t* buf,
                           auto defer) __attribute__((always_inline)) {
    // Not unrolled: unrolling lets the compiler hoist every tile's LDS reads
    // (32 registers each) ahead of the first pair's math, and spill.
#pragma unroll 1
    for (int tt = 0; tt < kStageTiles; tt += 2) {
      const int t = st * kStageTiles + tt;
      if (t >= ntiles) break;  // wave-uniform; the rest of the stage is past this wave's keys
      if (t + 1 < tbeg) continue;  // wave-uniform; both tiles precede this wave's window
      bool ok_a = true, ok_b = true;
      if constexpr (decltype(masked)::value && kPaged) {
        ok_a = key_ok<kPaged>(P, bt_row, t * kTile, kh, vh, pc);
        ok_b = key_ok<kPaged>(P, bt_row, (t + 1) * kTile, kh, vh, pc);
      }
      if constexpr (decltype(defer)::value) {
        pend_vm = pair_scores(masked, t * kTile, buf, tt, ok_a, ok_b, pend_pa, pend_pb,
                              std::false_type{});
        pend = true;
        pend_tok0 = t * kTile;
        pend_buf = buf;
        pend_ok_a = ok_a;
        pend_ok_b = ok_b;
      } else {
        short4_t p_a[kCB], p_b[kCB];
        const bool vm =
            pair_scores(masked, t * kTile, buf, tt, ok_a, ok_b, p_a, p_b, std::true_type{});
        pair_pv(t * kTile, buf, tt, ok_a, ok_b, vm, p_a, p_b, std::true_type{});
      }
    }
  };
  auto run_pending = [&]() __attribute__((always_inline)) {
    if (pend)
      pair_pv(pend_tok0, pend_buf, 0, pend_ok_a, pend_ok_b, pend_vm, pend_pa, pend_pb,
              std::false_type{});
    pend = false;
  };
  // A stage needs no mask when this wave sees all its keys in full (its tiles
  // below nfull: stages below un_full) and none of its pages is masked (below
  // ok_until; stage st is staged before step(st) tests it); under a window it
  // also starts at or after khead, which every stage after the masked head does.
  const int un_full = nfull / kStageTiles;
  auto stage_unmasked = [&](int st) { return st < min(un_full, ok_until); };
  // kConv: stage st's fp8 rows into its bf16 buffer, the chunks spread over the
  // threads of the half.  fp8 chunk q of a row (dims 16q .. 16q + 15) becomes
  // bf16 chunks 2q and 2q + 1 of the row, in the bf16 stage layout.
  auto stage_convert = [&](int st) {
    if constexpr (kConv || kConv1) {
      static_assert(S::kKChunks == S::kVChunks && S::kKChunks == S::kKReal, "fp8: D = DV");
      constexpr int kRowChunks = S::kNK;  // fp8 chunks of K (or V)
      constexpr int kThreads = kPrefillWaves * 64;
      const uint8_t* fbuf = stage_buf(st);
      uint8_t* bbuf = comp_buf(st);
      const int tid = threadIdx.x & (kThreads - 1);
#pragma unroll
      for (int c0 = 0; c0 < 2 * kRowChunks; c0 += kThreads) {
        const int c = c0 + tid;
        const int which = c / kRowChunks;  // 0: K, 1: V
        const int rem = c - which * kRowChunks;
        const int row = rem / S::kKChunks;
        const int q = rem - row * S::kKChunks;
        const uint4 x = *reinterpret_cast<const uint4*>(fbuf + S::offset(which, row, q));
        const float sc = which ? vsc : ks;
        const uint2 a = fp8x4_to_bf16x4(x.x, sc), b = fp8x4_to_bf16x4(x.y, sc);
        const uint2 e = fp8x4_to_bf16x4(x.z, sc), f = fp8x4_to_bf16x4(x.w, sc);
        *reinterpret_cast<uint4*>(bbuf + SB::offset(which, row, 2 * q)) = make_uint4(a.x, a.y, b.x, b.y);
        *reinterpret_cast<uint4*>(bbuf + SB::offset(which, row, 2 * q + 1)) =
            make_uint4(e.x, e.y, f.x, f.y);
      }
    }
  };
  // One step: wait for stage st's loads (every thread's, through the barrier,
  // which also frees the buffer the next loads go to), issue stage st + 1's,
  // consume stage st.  The unmasked and masked stages run in separate loops;
  // every wave passes exactly nsteps barriers whichever loops it is in.
  // kConv: stage st + 1's loads landed (the wait and the barrier), so it is
  // converted, and stage st + 2 is staged into the fp8 buffer stage st held
  // (converted in the step before); stage st is read from its bf16 buffer.
  auto step = [&](auto masked, int st, auto defer) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if constexpr (decltype(defer)::value) run_pending();
    if constexpr (kKEarly && !decltype(masked)::value && !decltype(defer)::value) {
      lds_k_chunks<D, DV>(comp_buf(st), 0, r, g, kpre);
      kpre_ok = true;
    }
    if constexpr (kConv) {
      if (st + 1 < st_hi) stage_convert(st + 1);
      if (st + 2 < st_hi) stage_load(st + 2);
    } else if constexpr (!kConv1) {
      if (st + 1 < st_hi) stage_load(st + 1);
    }
    stage_compute(masked, st, comp_buf(st), defer);
    kpre_ok = false;
    if constexpr (kConv1) {
      __syncthreads();  // every wave is done with the bf16 buffer
      if (st + 1 < st_hi) stage_convert(st + 1);
      if (st + 2 < st_hi) stage_load(st + 2);
    }
  };
  // Stages [st0, nstages): under a window, a masked head (keys some query's
  // window starts after), then the unmasked stages, then the masked rest.
  if (st_lo < st_hi) stage_load(st_lo);
  if constexpr (kConv || kConv1) {
    // The first stage converted before the loop, the second staged; every wave
    // of the work-group passes this barrier (with the key split the halves'
    // ranges differ, one may be empty).
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (st_lo < st_hi) stage_convert(st_lo);
    if (st_lo + 1 < st_hi) stage_load(st_lo + 1);
  }
  const int head_end = win >= 0 ? max(st0, (khead + kStageKeys - 1) / kStageKeys) : st0;
  auto run_stages = [&](auto defer) __attribute__((always_inline)) {
    int st = st_lo;
#pragma unroll 1
    for (; st < st_hi && st < head_end; ++st) step(std::true_type{}, st, defer);
#pragma unroll 1
    for (; st < st_hi && stage_unmasked(st); ++st) step(std::false_type{}, st, defer);
#pragma unroll 1
    for (; st < st_hi; ++st) step(std::true_type{}, st, defer);
    if constexpr (decltype(defer)::value) run_pending();
  };
  if constexpr (kPingPong) {
    if (half == 1)
      run_stages(std::true_type{});
    else
      run_stages(std::false_type{});
  } else {
    run_stages(std::false_type{});
  }
  // kLse: the column's fp32 sum (every lane of column r gets it).
  if constexpr (kLse) {
#pragma unroll
    for (int nb = 0; nb < kCB; ++nb) l32[nb] = pair_sum(l32[nb]);
  }
  // Row maxima and sums of the rows this lane holds (row 4g + i of block nb).
  float m_row[kCB][4], l_row[kCB][4];
#pragma unroll
  for (int nb = 0; nb < kCB; ++nb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m_row[nb][i] = row_from(m_run[nb], g, i);
      l_row[nb][i] = l_acc[nb][i];
    }
  if (kKS > 1 && !solo) {
#pragma unroll 1
    for (int k = st_hi - st_lo; k < nsteps; ++k) {  // the shorter half's empty steps
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if constexpr (kConv1) __syncthreads();
    }
    __syncthreads();  // every wave is done with the stage buffers
    // Exchange area of this wave role: O tiles, row sums, column maxima.
    float* const xo = reinterpret_cast<float*>(lds_all) + wave * kXFloats;
    float* const xl = xo + kCB * kVS * 64 * 4;
    float* const xm = xl + kCB * 64 * 4;
    float* const x32 = xm + kCB * 64;  // kLse: the columns' fp32 sums
    if (half == 1 && active) {
#pragma unroll
      for (int nb = 0; nb < kCB; ++nb) {
#pragma unroll
        for (int d = 0; d < kVS; ++d)
          *reinterpret_cast<floatx4_t*>(xo + ((nb * kVS + d) * 64 + lane) * 4) = o[nb][d];
        *reinterpret_cast<floatx4_t*>(xl + (nb * 64 + lane) * 4) = l_acc[nb];
        xm[nb * 64 + lane] = m_run[nb];
        if constexpr (kLse) x32[nb * 64 + lane] = l32[nb];
      }
    }
    __syncthreads();
    if (half == 1) return;  // from process_block: the first half writes the rows
    if (active) {
      // Log-sum-exp merge of the two halves, row by row (reduce_segments'
      // rule): M = max(m_a, m_b), O = O_a 2^(m_a - M) + O_b 2^(m_b - M), and
      // the same for the sums; a half that saw no key (max -inf) weighs 0.
#pragma unroll
      for (int nb = 0; nb < kCB; ++nb) {
        const float mb_col = xm[nb * 64 + lane];
        const floatx4_t lb = *reinterpret_cast<const floatx4_t*>(xl + (nb * 64 + lane) * 4);
        if constexpr (kLse) {  // the same merge for the columns' fp32 sums
          const float ma = m_run[nb];
          const float mx = fmaxf(ma, mb_col);
          const float wa = ma == kNegInf ? 0.f : __builtin_amdgcn_exp2f(ma - mx);
          const float wb = mb_col == kNegInf ? 0.f : __builtin_amdgcn_exp2f(mb_col - mx);
          l32[nb] = l32[nb] * wa + x32[nb * 64 + lane] * wb;
          m_run[nb] = mx;
        }
        float wa[4], wb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ma = m_row[nb][i];
          const float mb = row_from(mb_col, g, i);
          const float mx = fmaxf(ma, mb);
          wa[i] = ma == kNegInf ? 0.f : __builtin_amdgcn_exp2f(ma - mx);
          wb[i] = mb == kNegInf ? 0.f : __builtin_amdgcn_exp2f(mb - mx);
          m_row[nb][i] = mx;
          l_row[nb][i] = l_row[nb][i] * wa[i] + lb[i] * wb[i];
        }
#pragma unroll
        for (int d = 0; d < kVS; ++d) {
          const floatx4_t ob =
              *reinterpret_cast<const floatx4_t*>(xo + ((nb * kVS + d) * 64 + lane) * 4);
#pragma unroll
          for (int i = 0; i < 4; ++i) o[nb][d][i] = o[nb][d][i] * wa[i] + ob[i] * wb[i];
        }
      }
    }
  }
  if (!active) return;  // from process_block: this wave has no queries here

  // Work-group key split: this part's state (O before the division, the row's
  // max and sum) for prefill_merge_kernel, which applies the sink and writes the
  // rows and the log-sum-exp.  Every part writes every row of its block, also
  // one that saw no key (max -inf, sum 0).
  if (xs > 1) {
    const int64_t prow0 = static_cast<int64_t>(xpart) * P.part_rows + q_start;
    uint16_t* const part_o = static_cast<uint16_t*>(P.part);
    float* const part_ml = reinterpret_cast<float*>(
        static_cast<uint8_t*>(P.part) + part_ml_offset(xs, P.part_rows, P.num_heads, DV));
#pragma unroll
    for (int nb = 0; nb < kCB; ++nb) {
      if constexpr (kLse) {  // column layout: lanes of row group 0 hold column r's sum
        const int jc = j0 + 16 * nb + r;
        if (g == 0 && jc < q_len)
          part_ml[((prow0 + jc) * P.num_heads + hq) * kPartMl + 2] = l32[nb];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int jr = j0 + 16 * nb + 4 * g + i;
        if (jr >= q_len) continue;
        const int64_t rh = (prow0 + jr) * P.num_heads + hq;
        uint16_t* const po = part_o + rh * DV;
#pragma unroll
        for (int d = 0; d < kVS; ++d) {
          const int dim = kFp8T ? (D / 16) * r + d : 16 * d + r;
          if (kFp8T ? dim < DV : (16 * d + 16 <= DV || dim < DV))
            po[dim] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(o[nb][d][i]));
        }
        if (r == 0) {
          float* const pm = part_ml + rh * kPartMl;
          pm[0] = m_row[nb][i];
          pm[1] = l_row[nb][i];
        }
      }
    }
    return;
  }

  // kLse: lse = ln(sum e^(scale q.k)) = (m + log2 l) ln 2 per query column, the
  // sink included; -inf for a row with no visible key.  Lanes of row group 0
  // (r = column) write it.
  if constexpr (kLse) {
#pragma unroll
    for (int nb = 0; nb < kCB; ++nb) {
      const int jc = j0 + 16 * nb + r;
      float l = l32[nb];
      if (P.sinks) l = with_sink(l, m_run[nb], P.sinks[hq] * kLog2e);
      if (g == 0 && jc < q_len)
        P.lse[hq * P.lse_row_stride + q_start + jc] =
            l > 0.f ? (m_run[nb] + __log2f(l)) * 0.6931471805599453f : kNegInf;
    }
  }

#pragma unroll
  for (int nb = 0; nb < kCB; ++nb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int jr = j0 + 16 * nb + 4 * g + i;  // query row this lane holds
      float l = l_row[nb][i];
      if (P.sinks) l = with_sink(l, m_row[nb][i], P.sinks[hq] * kLog2e);
      if (jr >= q_len) continue;
      const float f = l > 0.f ? 1.f / l : 0.f;
      uint16_t* orow = P.out + static_cast<int64_t>(q_start + jr) * P.out_row_stride +
                       static_cast<int64_t>(hq) * DV;
      if constexpr (!kFp8T) {
        // o[nb][d] holds dim 16d + r: lanes r = 0..15 write 16 adjacent dims (the
        // padding dims past DV are not written).
#pragma unroll
        for (int d = 0; d < kVS; ++d)
          if (16 * d + 16 <= DV || 16 * d + r < DV)
            orow[16 * d + r] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(o[nb][d][i] * f));
      } else {
        // o[nb][d] holds dim (D/16) r + d: D/16 adjacent dims per lane.
        uint32_t w[D / 32];
#pragma unroll
        for (int d = 0; d < D / 32; ++d) {
          const bf16x2_t pk = {static_cast<__bf16>(o[nb][2 * d][i] * f),
                               static_cast<__bf16>(o[nb][2 * d + 1][i] * f)};
          w[d] = __builtin_bit_cast(uint32_t, pk);
        }
        uint16_t* dst = orow + (D / 16) * r;
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
  }
  };
  const int heavy = nqb - 1 - x;
  // Key split over a causal pair (kSplitPair): the first half streams the head of
  // the heavy block; the second half streams the whole light block and writes its
  // rows (no merge), then the heavy block's tail; the halves then merge the heavy
  // block.  Each half passes T step barriers (the shorter pads with empty steps)
  // and the merge's two barriers.  The second half's heavy stages start in the
  // buffer the light block's next stage would have used: every wave of the half
  // is past the light block's last barrier by then, and that buffer held a stage
  // at least two steps old.
  const bool split_pair = kSplitPair && paired && x != heavy;
  int s0l = 0, lol = 0, hil = 0, s0h = 0, loh = 0, hih = 0, sp_a = 0, sp_t = 0;
  if (split_pair) {
    wg_range(x, s0l, lol, hil);
    wg_range(heavy, s0h, loh, hih);
    const int nl = hil - lol, nh = hih - loh;
    const int a0 = (kPingPong && kDQ > 64) ? (nh + nl + 2) / 2 : (nh + nl + 1) / 2;
    sp_a = min(nh, a0);                   // the heavy block's stages of the first half
    sp_t = max(sp_a, nl + nh - sp_a);     // step barriers per half
  }
  // Odd work-groups of a paired launch (4-wave work-groups) take their light block
  // first (FK_PREFILL_ALT_ORDER), so that the two work-groups a CU holds (the same
  // work each) reach their block change at different times instead of stalling
  // together.
  const bool light_first = FK_PREFILL_ALT_ORDER && kKS == 1 && paired && (x & 1);
  if constexpr (kSplitPair) {
    // The blocks this half takes, in order: one loop and one call site, so that
    // the block code is emitted once (an instance per call site tripled the
    // kernel's code, 37 -> 140 KB).
    const int nseg = split_pair ? (half == 0 ? 1 : 2) : ((paired && x != heavy) ? 2 : 1);
#pragma unroll 1
    for (int k = 0; k < nseg; ++k) {
      int qblk, st0, st_lo, st_hi, nsteps;
      bool solo = false;
      if (split_pair) {
        if (half == 0) {
          qblk = heavy, st0 = s0h, st_lo = loh, st_hi = loh + sp_a, nsteps = sp_t;
        } else if (k == 0) {
          qblk = x, st0 = s0l, st_lo = lol, st_hi = hil, nsteps = hil - lol, solo = true;
        } else {
          qblk = heavy, st0 = s0h, st_lo = loh + sp_a, st_hi = hih,
          nsteps = sp_t - (hil - lol);
          buf_rot = ((hil - st_lo) % kBufs + kBufs) % kBufs;
        }
      } else {
        if (k == 1) __syncthreads();  // every wave is done with the last stage buffer
        qblk = k == 0 ? heavy : x;
        stage_range(qblk, st0, st_lo, st_hi, nsteps);
      }
      process_block(qblk, st0, st_lo, st_hi, nsteps, solo);
    }
  } else {
    // A loop rather than two calls: one copy of the block code (registers).
#pragma unroll 1
    for (int k = 0; k < 2; ++k) {
      if (k == 1) {
        if (!paired || x == heavy) break;  // unpaired, or the middle block of an odd count
        __syncthreads();                   // every wave is done with the last stage buffer
      }
      const int qblk = (k == 0) != light_first ? heavy : x;
      int st0, st_lo, st_hi, nsteps;
      stage_range(qblk, st0, st_lo, st_hi, nsteps);
      process_block(qblk, st0, st_lo, st_hi, nsteps, false);
    }
  }
}

// Whether the key split (8-wave work-groups) is built for these head sizes.
constexpr bool prefill_can_split(int D, int DV, bool paged) {
  return (D > DV ? D : DV) <= 192 || paged;
}

template <bool FP8, bool PAGED, int D, int DV, bool LSE>
void launch_prefill_lse(bool split, const PrefillParams& P, dim3 grid, const int32_t* bt,
                        const int32_t* cu_q, const int32_t* cu_k, hipStream_t stream) {
  if constexpr (prefill_can_split(D, DV, PAGED)) {
    if (split) {
      hipLaunchKernelGGL((paged_prefill_kernel<FP8, PAGED, D, DV, 2, LSE>), grid,
                         dim3(2 * kPrefillWaves * 64), 0, stream, P, bt, cu_q, cu_k);
      return;
    }
  }
  hipLaunchKernelGGL((paged_prefill_kernel<FP8, PAGED, D, DV, 1, LSE>), grid,
                     dim3(kPrefillWaves * 64), 0, stream, P, bt, cu_q, cu_k);
}

// The log-sum-exp output is built for dense keys (FlashAttnVarlen's
// return_softmax_lse); the entry point refuses it with paged keys.
template <bool FP8, bool PAGED, int D, int DV>
void launch_prefill(bool split, const PrefillParams& P, dim3 grid, const int32_t* bt,
                    const int32_t* cu_q, const int32_t* cu_k, hipStream_t stream) {
  if constexpr (!PAGED) {
    if (P.lse) {
      launch_prefill_lse<FP8, PAGED, D, DV, true>(split, P, grid, bt, cu_q, cu_k, stream);
      return;
    }
  }
  launch_prefill_lse<FP8, PAGED, D, DV, false>(split, P, grid, bt, cu_q, cu_k, stream);
}

// bf16 pages or dense keys (fp8 pages only where the template allows them).
template <int D, int DV>
void launch_prefill_bf16(bool paged, bool split, const PrefillParams& P, dim3 grid,
                         const int32_t* bt, const int32_t* cu_q, const int32_t* cu_k,
                         hipStream_t stream) {
  if (!paged)
    launch_prefill<false, false, D, DV>(split, P, grid, nullptr, cu_q, cu_k, stream);
  else
    launch_prefill<false, true, D, DV>(split, P, grid, bt, cu_q, cu_k, stream);
}

}  // namespace
}  // namespace fk
