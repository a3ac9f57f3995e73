// store_kvcache: bit-exact scatter of each token's K and V row into the NHD
// paged cache at slot_mapping[token] (fastkernels/tasks/baseline/L1/
// store_kvcache.py:16-35 computes the same mapping, one Triton program per token).
//
// MI355X layout: a token row is num_kv_heads*head_size contiguous elements
// (2 KiB for 8x128 bf16), and slot s owns bytes [s*row, (s+1)*row) of each cache.
// Each lane moves 16-byte chunks (global_load/store_dwordx4); a 256-lane
// work-group covers 256/chunks_per_row tokens, so one wave writes a contiguous
// 1 KiB run of a destination row and every access is a full 64-byte segment.
#include "fk_common.h"

namespace fk {
namespace {

template <typename IdxT>
__device__ __forceinline__ int64_t load_slot(const void* slot_mapping, int64_t i) {
  return static_cast<int64_t>(static_cast<const IdxT*>(slot_mapping)[i]);
}

// Vector path: row bytes, row strides and base pointers are multiples of 16 B.
template <typename IdxT>
__global__ __launch_bounds__(256) void store_kvcache_vec16(
    const uint4* __restrict__ key, int64_t key_row_chunks, const uint4* __restrict__ value,
    int64_t value_row_chunks, uint4* __restrict__ k_cache, uint4* __restrict__ v_cache,
    const void* __restrict__ slot_mapping, int64_t tokens, int chunks_per_row,
    int tokens_per_block, int64_t num_slots) {
  const int lane_tok = threadIdx.x / chunks_per_row;  // chunks_per_row <= 256 here
  const int chunk0 = threadIdx.x % chunks_per_row;
  if (lane_tok >= tokens_per_block) return;
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * tokens_per_block + lane_tok;
  if (tok >= tokens) return;
  // The source rows do not depend on the slot: issue their loads together with
  // the slot load so the kernel waits one memory round trip, not two.
  const uint4 kv = key[tok * key_row_chunks + chunk0];
  const uint4 vv = value[tok * value_row_chunks + chunk0];
  const int64_t slot = load_slot<IdxT>(slot_mapping, tok);
  if (slot < 0 || slot >= num_slots) return;
  k_cache[slot * chunks_per_row + chunk0] = kv;
  v_cache[slot * chunks_per_row + chunk0] = vv;
}

// Wide rows (> 256 chunks): one work-group per token, lanes stride the row.
template <typename IdxT>
__global__ __launch_bounds__(256) void store_kvcache_vec16_wide(
    const uint4* __restrict__ key, int64_t key_row_chunks, const uint4* __restrict__ value,
    int64_t value_row_chunks, uint4* __restrict__ k_cache, uint4* __restrict__ v_cache,
    const void* __restrict__ slot_mapping, int64_t tokens, int64_t chunks_per_row,
    int64_t num_slots) {
  const int64_t tok = blockIdx.x;
  const int64_t slot = load_slot<IdxT>(slot_mapping, tok);
  if (slot < 0 || slot >= num_slots) return;
  const uint4* ksrc = key + tok * key_row_chunks;
  const uint4* vsrc = value + tok * value_row_chunks;
  uint4* kdst = k_cache + slot * chunks_per_row;
  uint4* vdst = v_cache + slot * chunks_per_row;
  for (int64_t c = threadIdx.x; c < chunks_per_row; c += 256) {
    const uint4 kv = ksrc[c];
    const uint4 vv = vsrc[c];
    kdst[c] = kv;
    vdst[c] = vv;
  }
}

// Scalar path for any alignment: elements of ElemT (1, 2 or 4 bytes).
template <typename IdxT, typename ElemT>
__global__ __launch_bounds__(256) void store_kvcache_scalar(
    const ElemT* __restrict__ key, int64_t key_row_stride, const ElemT* __restrict__ value,
    int64_t value_row_stride, ElemT* __restrict__ k_cache, ElemT* __restrict__ v_cache,
    const void* __restrict__ slot_mapping, int64_t row_elems, int64_t num_slots) {
  const int64_t tok = blockIdx.x;
  const int64_t slot = load_slot<IdxT>(slot_mapping, tok);
  if (slot < 0 || slot >= num_slots) return;
  for (int64_t c = threadIdx.x; c < row_elems; c += 256) {
    k_cache[slot * row_elems + c] = key[tok * key_row_stride + c];
    v_cache[slot * row_elems + c] = value[tok * value_row_stride + c];
  }
}

template <typename IdxT>
int launch(const void* key, int64_t key_row_stride, const void* value, int64_t value_row_stride,
           void* k_cache, void* v_cache, const void* slot_mapping, int64_t tokens,
           int64_t row_elems, int elem_bytes, int64_t num_slots, hipStream_t stream) {
  const int64_t row_bytes = row_elems * elem_bytes;
  const bool vec = (row_bytes % 16 == 0) && ((key_row_stride * elem_bytes) % 16 == 0) &&
                   ((value_row_stride * elem_bytes) % 16 == 0) && aligned16(key) &&
                   aligned16(value) && aligned16(k_cache) && aligned16(v_cache);
  if (vec) {
    const int64_t cpr = row_bytes / 16;
    const int64_t krc = key_row_stride * elem_bytes / 16;
    const int64_t vrc = value_row_stride * elem_bytes / 16;
    if (cpr <= 256) {
      const int tpb = static_cast<int>(256 / cpr);
      const int64_t blocks = (tokens + tpb - 1) / tpb;
      hipLaunchKernelGGL(store_kvcache_vec16<IdxT>, dim3(static_cast<unsigned>(blocks)), dim3(256),
                         0, stream, static_cast<const uint4*>(key), krc,
                         static_cast<const uint4*>(value), vrc, static_cast<uint4*>(k_cache),
                         static_cast<uint4*>(v_cache), slot_mapping, tokens,
                         static_cast<int>(cpr), tpb, num_slots);
    } else {
      hipLaunchKernelGGL(store_kvcache_vec16_wide<IdxT>, dim3(static_cast<unsigned>(tokens)),
                         dim3(256), 0, stream, static_cast<const uint4*>(key), krc,
                         static_cast<const uint4*>(value), vrc, static_cast<uint4*>(k_cache),
                         static_cast<uint4*>(v_cache), slot_mapping, tokens, cpr, num_slots);
    }
    return check_launch("fk_store_kvcache");
  }
  const dim3 grid(static_cast<unsigned>(tokens));
  switch (elem_bytes) {
    case 1:
      hipLaunchKernelGGL((store_kvcache_scalar<IdxT, uint8_t>), grid, dim3(256), 0, stream,
                         static_cast<const uint8_t*>(key), key_row_stride,
                         static_cast<const uint8_t*>(value), value_row_stride,
                         static_cast<uint8_t*>(k_cache), static_cast<uint8_t*>(v_cache),
                         slot_mapping, row_elems, num_slots);
      break;
    case 2:
      hipLaunchKernelGGL((store_kvcache_scalar<IdxT, uint16_t>), grid, dim3(256), 0, stream,
                         static_cast<const uint16_t*>(key), key_row_stride,
                         static_cast<const uint16_t*>(value), value_row_stride,
                         static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                         slot_mapping, row_elems, num_slots);
      break;
    default:
      hipLaunchKernelGGL((store_kvcache_scalar<IdxT, uint32_t>), grid, dim3(256), 0, stream,
                         static_cast<const uint32_t*>(key), key_row_stride,
                         static_cast<const uint32_t*>(value), value_row_stride,
                         static_cast<uint32_t*>(k_cache), static_cast<uint32_t*>(v_cache),
                         slot_mapping, row_elems, num_slots);
      break;
  }
  return check_launch("fk_store_kvcache");
}

}  // namespace
}  // namespace fk

extern "C" int fk_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                                int64_t value_row_stride, void* k_cache, void* v_cache,
                                const void* slot_mapping, int slot_is_i64, int64_t tokens,
                                int64_t row_elems, int elem_bytes, int64_t num_slots,
                                void* stream) {
  FK_REQUIRE(tokens >= 0 && row_elems >= 0 && num_slots >= 0,
             "fk_store_kvcache: negative size (tokens=%lld row_elems=%lld num_slots=%lld)",
             (long long)tokens, (long long)row_elems, (long long)num_slots);
  FK_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4,
             "fk_store_kvcache: elem_bytes must be 1, 2 or 4 (got %d)", elem_bytes);
  FK_REQUIRE(tokens <= 0x7fffffffLL, "fk_store_kvcache: too many tokens (%lld)",
             (long long)tokens);
  FK_REQUIRE(key_row_stride >= row_elems && value_row_stride >= row_elems,
             "fk_store_kvcache: row stride shorter than the row (%lld/%lld < %lld)",
             (long long)key_row_stride, (long long)value_row_stride, (long long)row_elems);
  if (tokens == 0 || row_elems == 0) return FK_OK;
  FK_REQUIRE(key && value && k_cache && v_cache && slot_mapping,
             "fk_store_kvcache: null pointer");
  hipStream_t s = fk::as_stream(stream);
  if (slot_is_i64)
    return fk::launch<int64_t>(key, key_row_stride, value, value_row_stride, k_cache, v_cache,
                               slot_mapping, tokens, row_elems, elem_bytes, num_slots, s);
  return fk::launch<int32_t>(key, key_row_stride, value, value_row_stride, k_cache, v_cache,
                             slot_mapping, tokens, row_elems, elem_bytes, num_slots, s);
}

// ---------------------------------------------------------------------------
// Store with a dtype conversion: the reference's Triton store writes a bf16 /
// fp16 / fp32 key into a cache of another dtype with tl.store's implicit cast
// (store_kvcache.py:32-35), which for a float8_e4m3fn cache rounds to nearest
// even and saturates to the largest finite value (+-448).
// ---------------------------------------------------------------------------
namespace fk {
namespace {

template <typename Src>
__device__ __forceinline__ float src_to_f32(typename Src::storage v) { return Src::to_f32(v); }

// Destination element from fp32, by cache dtype tag.
template <int kDst>
struct DstConv;
template <>
struct DstConv<FK_DTYPE_FP8_E4M3FN> {
  using storage = uint8_t;
  __device__ __forceinline__ static storage conv(float f) { return f32_to_e4m3fn_sat(f); }
};
template <>
struct DstConv<FK_DTYPE_BF16> {
  using storage = uint16_t;
  __device__ __forceinline__ static storage conv(float f) { return BF16::from_f32(f); }
};
template <>
struct DstConv<FK_DTYPE_F16> {
  using storage = uint16_t;
  __device__ __forceinline__ static storage conv(float f) { return F16::from_f32(f); }
};
template <>
struct DstConv<FK_DTYPE_F32> {
  using storage = float;
  __device__ __forceinline__ static storage conv(float f) { return f; }
};

// One work-group per token; lanes stride the row element by element (the
// conversion store is not on the decode step's hot path: the bf16 cache uses
// the bit-copy kernels above).
template <typename IdxT, typename Src, int kDst>
__global__ __launch_bounds__(256) void store_kvcache_convert(
    const typename Src::storage* __restrict__ key, int64_t key_row_stride,
    const typename Src::storage* __restrict__ value, int64_t value_row_stride,
    typename DstConv<kDst>::storage* __restrict__ k_cache,
    typename DstConv<kDst>::storage* __restrict__ v_cache, const void* __restrict__ slot_mapping,
    int64_t row_elems, int64_t num_slots) {
  const int64_t tok = blockIdx.x;
  const int64_t slot = load_slot<IdxT>(slot_mapping, tok);
  if (slot < 0 || slot >= num_slots) return;
  for (int64_t c = threadIdx.x; c < row_elems; c += 256) {
    k_cache[slot * row_elems + c] = DstConv<kDst>::conv(Src::to_f32(key[tok * key_row_stride + c]));
    v_cache[slot * row_elems + c] =
        DstConv<kDst>::conv(Src::to_f32(value[tok * value_row_stride + c]));
  }
}

template <typename IdxT, typename Src, int kDst>
int launch_convert(const void* key, int64_t key_row_stride, const void* value,
                   int64_t value_row_stride, void* k_cache, void* v_cache,
                   const void* slot_mapping, int64_t tokens, int64_t row_elems, int64_t num_slots,
                   hipStream_t stream) {
  using S = typename Src::storage;
  using D = typename DstConv<kDst>::storage;
  hipLaunchKernelGGL((store_kvcache_convert<IdxT, Src, kDst>), dim3(static_cast<unsigned>(tokens)),
                     dim3(256), 0, stream, static_cast<const S*>(key), key_row_stride,
                     static_cast<const S*>(value), value_row_stride, static_cast<D*>(k_cache),
                     static_cast<D*>(v_cache), slot_mapping, row_elems, num_slots);
  return check_launch("fk_store_kvcache_convert");
}

template <typename IdxT, typename Src>
int convert_dst(int cache_dtype, const void* key, int64_t ks, const void* value, int64_t vs,
                void* kc, void* vc, const void* sm, int64_t tokens, int64_t row, int64_t slots,
                hipStream_t s) {
  switch (cache_dtype) {
    case FK_DTYPE_FP8_E4M3FN:
      return launch_convert<IdxT, Src, FK_DTYPE_FP8_E4M3FN>(key, ks, value, vs, kc, vc, sm, tokens,
                                                             row, slots, s);
    case FK_DTYPE_BF16:
      return launch_convert<IdxT, Src, FK_DTYPE_BF16>(key, ks, value, vs, kc, vc, sm, tokens, row,
                                                       slots, s);
    case FK_DTYPE_F16:
      return launch_convert<IdxT, Src, FK_DTYPE_F16>(key, ks, value, vs, kc, vc, sm, tokens, row,
                                                      slots, s);
    case FK_DTYPE_F32:
      return launch_convert<IdxT, Src, FK_DTYPE_F32>(key, ks, value, vs, kc, vc, sm, tokens, row,
                                                      slots, s);
    default:
      return set_error(FK_ERR_UNSUPPORTED, "fk_store_kvcache_convert: cache dtype %d unsupported",
                       cache_dtype);
  }
}

template <typename IdxT>
int convert_src(int src_dtype, int cache_dtype, const void* key, int64_t ks, const void* value,
                int64_t vs, void* kc, void* vc, const void* sm, int64_t tokens, int64_t row,
                int64_t slots, hipStream_t s) {
  switch (src_dtype) {
    case FK_DTYPE_BF16:
      return convert_dst<IdxT, BF16>(cache_dtype, key, ks, value, vs, kc, vc, sm, tokens, row,
                                     slots, s);
    case FK_DTYPE_F16:
      return convert_dst<IdxT, F16>(cache_dtype, key, ks, value, vs, kc, vc, sm, tokens, row,
                                    slots, s);
    case FK_DTYPE_F32:
      return convert_dst<IdxT, F32>(cache_dtype, key, ks, value, vs, kc, vc, sm, tokens, row,
                                    slots, s);
    default:
      return set_error(FK_ERR_UNSUPPORTED, "fk_store_kvcache_convert: key dtype %d unsupported",
                       src_dtype);
  }
}

}  // namespace
}  // namespace fk

extern "C" int fk_store_kvcache_convert(const void* key, int64_t key_row_stride,
                                        const void* value, int64_t value_row_stride,
                                        int src_dtype, void* k_cache, void* v_cache,
                                        int cache_dtype, const void* slot_mapping,
                                        int slot_is_i64, int64_t tokens, int64_t row_elems,
                                        int64_t num_slots, void* stream) {
  FK_REQUIRE(tokens >= 0 && row_elems >= 0 && num_slots >= 0,
             "fk_store_kvcache_convert: negative size");
  FK_REQUIRE(tokens <= 0x7fffffffLL, "fk_store_kvcache_convert: too many tokens");
  FK_REQUIRE(key_row_stride >= row_elems && value_row_stride >= row_elems,
             "fk_store_kvcache_convert: row stride shorter than the row");
  if (tokens == 0 || row_elems == 0) return FK_OK;
  FK_REQUIRE(key && value && k_cache && v_cache && slot_mapping,
             "fk_store_kvcache_convert: null pointer");
  hipStream_t s = fk::as_stream(stream);
  if (slot_is_i64)
    return fk::convert_src<int64_t>(src_dtype, cache_dtype, key, key_row_stride, value,
                                    value_row_stride, k_cache, v_cache, slot_mapping, tokens,
                                    row_elems, num_slots, s);
  return fk::convert_src<int32_t>(src_dtype, cache_dtype, key, key_row_stride, value,
                                  value_row_stride, k_cache, v_cache, slot_mapping, tokens,
                                  row_elems, num_slots, s);
}

// ---------------------------------------------------------------------------
// HND layout: StoreKVCacheHND (store_kvcache.py:36-99) writes token i's head h
// row to cache[slot / page][h][slot % page][:] of a
// [num_blocks, num_kv_heads, page_size, head_size] cache, so one token's heads
// land page_size * head_size elements apart.  A lane moves one 16-byte chunk; a
// (token, head) row of cpr chunks is handled by cpr consecutive lanes.
// ---------------------------------------------------------------------------
namespace fk {
namespace {

template <typename IdxT>
__global__ __launch_bounds__(256) void store_kvcache_hnd_vec16(
    const uint4* __restrict__ key, int64_t key_row_chunks, const uint4* __restrict__ value,
    int64_t value_row_chunks, uint4* __restrict__ k_cache, uint4* __restrict__ v_cache,
    const void* __restrict__ slot_mapping, int64_t rows, int num_kv_heads, int cpr,
    int page_size, int64_t num_slots) {
  const int64_t lin = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = lin / cpr;  // (token, head) row
  if (row >= rows) return;
  const int c = static_cast<int>(lin - row * cpr);
  const int64_t tok = row / num_kv_heads;
  const int h = static_cast<int>(row - tok * num_kv_heads);
  // Source loads first, independent of the slot, so the wait is one round trip.
  const uint4 kv = key[tok * key_row_chunks + static_cast<int64_t>(h) * cpr + c];
  const uint4 vv = value[tok * value_row_chunks + static_cast<int64_t>(h) * cpr + c];
  const int64_t slot = load_slot<IdxT>(slot_mapping, tok);
  if (slot < 0 || slot >= num_slots) return;
  const int64_t blk = slot / page_size;
  const int64_t dst = ((blk * num_kv_heads + h) * page_size + (slot - blk * page_size)) * cpr + c;
  k_cache[dst] = kv;
  v_cache[dst] = vv;
}

template <typename IdxT, typename ElemT>
__global__ __launch_bounds__(256) void store_kvcache_hnd_scalar(
    const ElemT* __restrict__ key, int64_t key_row_stride, const ElemT* __restrict__ value,
    int64_t value_row_stride, ElemT* __restrict__ k_cache, ElemT* __restrict__ v_cache,
    const void* __restrict__ slot_mapping, int num_kv_heads, int head_size, int page_size,
    int64_t num_slots) {
  const int64_t tok = blockIdx.x;
  const int h = blockIdx.y;
  const int64_t slot = load_slot<IdxT>(slot_mapping, tok);
  if (slot < 0 || slot >= num_slots) return;
  const int64_t blk = slot / page_size;
  const int64_t dst = ((blk * num_kv_heads + h) * page_size + (slot - blk * page_size)) * head_size;
  for (int e = threadIdx.x; e < head_size; e += 256) {
    k_cache[dst + e] = key[tok * key_row_stride + static_cast<int64_t>(h) * head_size + e];
    v_cache[dst + e] = value[tok * value_row_stride + static_cast<int64_t>(h) * head_size + e];
  }
}

template <typename IdxT>
int launch_hnd(const void* key, int64_t ks, const void* value, int64_t vs, void* kc, void* vc,
               const void* sm, int64_t tokens, int hk, int head_size, int page_size,
               int elem_bytes, int64_t num_slots, hipStream_t stream) {
  const int64_t head_bytes = static_cast<int64_t>(head_size) * elem_bytes;
  const bool vec = head_bytes % 16 == 0 && (ks * elem_bytes) % 16 == 0 &&
                   (vs * elem_bytes) % 16 == 0 && aligned16(key) && aligned16(value) &&
                   aligned16(kc) && aligned16(vc);
  if (vec) {
    const int cpr = static_cast<int>(head_bytes / 16);
    const int64_t rows = tokens * hk;
    const int64_t blocks = (rows * cpr + 255) / 256;
    FK_REQUIRE(blocks <= 0x7fffffffLL, "fk_store_kvcache_hnd: too many rows");
    hipLaunchKernelGGL(store_kvcache_hnd_vec16<IdxT>, dim3(static_cast<unsigned>(blocks)),
                       dim3(256), 0, stream, static_cast<const uint4*>(key), ks * elem_bytes / 16,
                       static_cast<const uint4*>(value), vs * elem_bytes / 16,
                       static_cast<uint4*>(kc), static_cast<uint4*>(vc), sm, rows, hk, cpr,
                       page_size, num_slots);
    return check_launch("fk_store_kvcache_hnd");
  }
  const dim3 grid(static_cast<unsigned>(tokens), static_cast<unsigned>(hk));
  switch (elem_bytes) {
    case 1:
      hipLaunchKernelGGL((store_kvcache_hnd_scalar<IdxT, uint8_t>), grid, dim3(256), 0, stream,
                         static_cast<const uint8_t*>(key), ks, static_cast<const uint8_t*>(value),
                         vs, static_cast<uint8_t*>(kc), static_cast<uint8_t*>(vc), sm, hk,
                         head_size, page_size, num_slots);
      break;
    case 2:
      hipLaunchKernelGGL((store_kvcache_hnd_scalar<IdxT, uint16_t>), grid, dim3(256), 0, stream,
                         static_cast<const uint16_t*>(key), ks,
                         static_cast<const uint16_t*>(value), vs, static_cast<uint16_t*>(kc),
                         static_cast<uint16_t*>(vc), sm, hk, head_size, page_size, num_slots);
      break;
    default:
      hipLaunchKernelGGL((store_kvcache_hnd_scalar<IdxT, uint32_t>), grid, dim3(256), 0, stream,
                         static_cast<const uint32_t*>(key), ks,
                         static_cast<const uint32_t*>(value), vs, static_cast<uint32_t*>(kc),
                         static_cast<uint32_t*>(vc), sm, hk, head_size, page_size, num_slots);
      break;
  }
  return check_launch("fk_store_kvcache_hnd");
}

}  // namespace
}  // namespace fk

extern "C" int fk_store_kvcache_hnd(const void* key, int64_t key_row_stride, const void* value,
                                    int64_t value_row_stride, void* k_cache, void* v_cache,
                                    const void* slot_mapping, int slot_is_i64, int64_t tokens,
                                    int num_kv_heads, int head_size, int page_size,
                                    int elem_bytes, int64_t num_slots, void* stream) {
  const char* name = "fk_store_kvcache_hnd";
  FK_REQUIRE(tokens >= 0 && num_kv_heads > 0 && head_size > 0 && num_slots >= 0,
             "%s: bad size (tokens=%lld heads=%d head_size=%d)", name, (long long)tokens,
             num_kv_heads, head_size);
  FK_REQUIRE(num_kv_heads <= 65535, "%s: too many kv heads (%d)", name, num_kv_heads);
  FK_REQUIRE(page_size > 0, "%s: page_size %d must be positive", name, page_size);
  FK_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4,
             "%s: elem_bytes must be 1, 2 or 4 (got %d)", name, elem_bytes);
  FK_REQUIRE(tokens <= 0x7fffffffLL, "%s: too many tokens (%lld)", name, (long long)tokens);
  const int64_t row = static_cast<int64_t>(num_kv_heads) * head_size;
  FK_REQUIRE(key_row_stride >= row && value_row_stride >= row,
             "%s: row stride shorter than num_kv_heads * head_size", name);
  if (tokens == 0) return FK_OK;
  FK_REQUIRE(key && value && k_cache && v_cache && slot_mapping, "%s: null pointer", name);
  hipStream_t s = fk::as_stream(stream);
  if (slot_is_i64)
    return fk::launch_hnd<int64_t>(key, key_row_stride, value, value_row_stride, k_cache, v_cache,
                                   slot_mapping, tokens, num_kv_heads, head_size, page_size,
                                   elem_bytes, num_slots, s);
  return fk::launch_hnd<int32_t>(key, key_row_stride, value, value_row_stride, k_cache, v_cache,
                                 slot_mapping, tokens, num_kv_heads, head_size, page_size,
                                 elem_bytes, num_slots, s);
}
