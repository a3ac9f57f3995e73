// Rotary position embedding, in place on query and key rows.
//
// Semantics follow RotaryEmbedding (fastkernels/tasks/baseline/L1/rotary_emb.py):
//   cos_sin_cache[p] = [cos(p * inv_freq), sin(p * inv_freq)]      (:104-107)
//   cos/sin are cast to the query dtype before use                 (:171-173)
//   NeoX (:110-139):   o[i]      = x[i] cos_i - x[i+r/2] sin_i
//                      o[i+r/2]  = x[i+r/2] cos_i + x[i] sin_i
//   GPT-J (:142-167):  o[2i]     = x[2i] cos_i - x[2i+1] sin_i
//                      o[2i+1]   = x[2i+1] cos_i + x[2i] sin_i
// The products and the sum are formed in fp32 and rounded once to the dtype.
//
// MI355X mapping: one work-group per token; each lane rotates a 16-byte vector
// of pair elements (8 bf16) of one head, reading the matching cos/sin vector.
// q and k are strided row views of the fused qkv buffer, so each token touches
// (Hq + Hk) * head_size contiguous elements of its own row.
#include "fk_common.h"

namespace fk {
namespace {

template <typename T, typename CT, bool kNeox>
__global__ __launch_bounds__(256) void rotary_vec(
    const int64_t* __restrict__ positions, typename T::storage* __restrict__ query,
    int64_t q_row_stride, typename T::storage* __restrict__ key, int64_t k_row_stride,
    const typename CT::storage* __restrict__ cos_sin, int64_t max_position, int num_heads,
    int num_kv_heads, int head_size, int rot_dim) {
  using V = Vec16<T>;
  using S = typename T::storage;
  constexpr int N = V::N;
  // Work items (16-byte vectors) per lane per pass: all of a pass's q/k loads are
  // issued together with the position load, so a token costs one round trip for
  // q/k and the position and one for cos/sin, not one per item.
  constexpr int kItems = 2;
  const int64_t tok = blockIdx.x;
  const int half = rot_dim / 2;
  // kNeox: a vector holds N consecutive first-half (or second-half) elements,
  // npv vectors cover the first half.  GPT-J: a vector holds N/2 whole pairs.
  const int npv = kNeox ? half / N : rot_dim / N;
  const int total = (num_heads + num_kv_heads) * npv;
  const int64_t pos = positions[tok];
  // No early exit on the position: the loads above and below stay independent of
  // it; an out-of-range position only suppresses the stores.
  const bool pos_ok = pos >= 0 && pos < max_position;
  const typename CT::storage* cs = cos_sin + (pos_ok ? pos : 0) * rot_dim;
  for (int w0 = threadIdx.x; w0 < total; w0 += 256 * kItems) {
    S* base[kItems];
    int i0[kItems];
    bool ok[kItems];
    V xv[kItems], yv[kItems];
#pragma unroll
    for (int u = 0; u < kItems; ++u) {
      const int w = w0 + 256 * u;
      ok[u] = w < total;
      const int wc = ok[u] ? w : w0;  // an idle slot re-reads the pass's first item
      const int head = wc / npv;
      const int pv = wc - head * npv;
      base[u] = head < num_heads
                    ? query + tok * q_row_stride + static_cast<int64_t>(head) * head_size
                    : key + tok * k_row_stride + static_cast<int64_t>(head - num_heads) * head_size;
      i0[u] = pv * N;
      xv[u].raw = *reinterpret_cast<const uint4*>(base[u] + i0[u]);
      if constexpr (kNeox) yv[u].raw = *reinterpret_cast<const uint4*>(base[u] + half + i0[u]);
    }
#pragma unroll
    for (int u = 0; u < kItems; ++u) {
      if constexpr (kNeox) {
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const float c = T::round(CT::to_f32(cs[i0[u] + e]));
          const float sn = T::round(CT::to_f32(cs[half + i0[u] + e]));
          const float x = T::to_f32(xv[u].e[e]);
          const float y = T::to_f32(yv[u].e[e]);
          xv[u].e[e] = T::from_f32(rope_x(x, y, c, sn));
          yv[u].e[e] = T::from_f32(rope_y(x, y, c, sn));
        }
        if (ok[u] && pos_ok) {
          *reinterpret_cast<uint4*>(base[u] + i0[u]) = xv[u].raw;
          *reinterpret_cast<uint4*>(base[u] + half + i0[u]) = yv[u].raw;
        }
      } else {
        // element offset i0; pairs (i0 + 2j, i0 + 2j + 1)
#pragma unroll
        for (int j = 0; j < N / 2; ++j) {
          const int i = i0[u] / 2 + j;
          const float c = T::round(CT::to_f32(cs[i]));
          const float sn = T::round(CT::to_f32(cs[half + i]));
          const float x = T::to_f32(xv[u].e[2 * j]);
          const float y = T::to_f32(xv[u].e[2 * j + 1]);
          xv[u].e[2 * j] = T::from_f32(rope_x(x, y, c, sn));
          xv[u].e[2 * j + 1] = T::from_f32(rope_y(x, y, c, sn));
        }
        if (ok[u] && pos_ok) *reinterpret_cast<uint4*>(base[u] + i0[u]) = xv[u].raw;
      }
    }
  }
}

// Any alignment / rotary width: one lane per rotated pair.
template <typename T, typename CT, bool kNeox>
__global__ __launch_bounds__(256) void rotary_scalar(
    const int64_t* __restrict__ positions, typename T::storage* __restrict__ query,
    int64_t q_row_stride, typename T::storage* __restrict__ key, int64_t k_row_stride,
    const typename CT::storage* __restrict__ cos_sin, int64_t max_position, int num_heads,
    int num_kv_heads, int head_size, int rot_dim) {
  const int64_t tok = blockIdx.x;
  const int64_t pos = positions[tok];
  if (pos < 0 || pos >= max_position) return;
  const int half = rot_dim / 2;
  const int total = (num_heads + num_kv_heads) * half;
  const typename CT::storage* cs = cos_sin + pos * rot_dim;
  for (int w = threadIdx.x; w < total; w += 256) {
    const int head = w / half;
    const int i = w - head * half;
    typename T::storage* base =
        head < num_heads ? query + tok * q_row_stride + static_cast<int64_t>(head) * head_size
                         : key + tok * k_row_stride +
                               static_cast<int64_t>(head - num_heads) * head_size;
    const int xi = kNeox ? i : 2 * i;
    const int yi = kNeox ? i + half : 2 * i + 1;
    const float c = T::round(CT::to_f32(cs[i]));
    const float s = T::round(CT::to_f32(cs[half + i]));
    const float x = T::to_f32(base[xi]);
    const float y = T::to_f32(base[yi]);
    base[xi] = T::from_f32(rope_x(x, y, c, s));
    base[yi] = T::from_f32(rope_y(x, y, c, s));
  }
}

template <typename T, typename CT>
int launch_tc(const int64_t* positions, void* query, int64_t q_row_stride, void* key,
              int64_t k_row_stride, const void* cos_sin, int64_t max_position, int64_t tokens,
              int num_heads, int num_kv_heads, int head_size, int rot_dim, bool neox,
              hipStream_t stream) {
  using S = typename T::storage;
  constexpr int N = Vec16<T>::N;
  const int64_t es = sizeof(S);
  const int hk = key ? num_kv_heads : 0;
  const bool vec = (neox ? (rot_dim / 2) % N == 0 : rot_dim % N == 0) &&
                   (head_size * es) % 16 == 0 && (q_row_stride * es) % 16 == 0 &&
                   (!key || (k_row_stride * es) % 16 == 0) && aligned16(query) &&
                   (!key || aligned16(key));
  const dim3 grid(static_cast<unsigned>(tokens));
  auto* q = static_cast<S*>(query);
  auto* k = static_cast<S*>(key);
  const auto* cs = static_cast<const typename CT::storage*>(cos_sin);
#define FK_ROPE(KERNEL, NEOX)                                                               \
  hipLaunchKernelGGL((KERNEL<T, CT, NEOX>), grid, dim3(256), 0, stream, positions, q,       \
                     q_row_stride, k, k_row_stride, cs, max_position, num_heads, hk,        \
                     head_size, rot_dim)
  if (vec) {
    if (neox) FK_ROPE(rotary_vec, true); else FK_ROPE(rotary_vec, false);
  } else {
    if (neox) FK_ROPE(rotary_scalar, true); else FK_ROPE(rotary_scalar, false);
  }
#undef FK_ROPE
  return check_launch("fk_rotary_embedding");
}

template <typename T>
int launch_t(int cache_dtype, const int64_t* positions, void* query, int64_t q_row_stride,
             void* key, int64_t k_row_stride, const void* cos_sin, int64_t max_position,
             int64_t tokens, int num_heads, int num_kv_heads, int head_size, int rot_dim,
             bool neox, hipStream_t stream) {
  if (cache_dtype == FK_DTYPE_F32)
    return launch_tc<T, F32>(positions, query, q_row_stride, key, k_row_stride, cos_sin,
                             max_position, tokens, num_heads, num_kv_heads, head_size, rot_dim,
                             neox, stream);
  if (cache_dtype == T::kDtype)
    return launch_tc<T, T>(positions, query, q_row_stride, key, k_row_stride, cos_sin,
                           max_position, tokens, num_heads, num_kv_heads, head_size, rot_dim,
                           neox, stream);
  return set_error(FK_ERR_UNSUPPORTED,
                   "fk_rotary_embedding: cos_sin dtype %d must be f32 or the query dtype %d",
                   cache_dtype, T::kDtype);
}

}  // namespace
}  // namespace fk

extern "C" int fk_rotary_embedding(const int64_t* positions, void* query, int64_t q_row_stride,
                                   void* key, int64_t k_row_stride, const void* cos_sin,
                                   int cache_dtype, int64_t max_position, int64_t tokens,
                                   int num_heads, int num_kv_heads, int head_size, int rot_dim,
                                   int is_neox, int dtype, void* stream) {
  FK_REQUIRE(tokens >= 0 && tokens <= 0x7fffffffLL, "fk_rotary_embedding: bad token count %lld",
             (long long)tokens);
  FK_REQUIRE(num_heads > 0 && head_size > 0 && (!key || num_kv_heads > 0),
             "fk_rotary_embedding: bad head counts (heads=%d kv_heads=%d head_size=%d)",
             num_heads, num_kv_heads, head_size);
  FK_REQUIRE(rot_dim > 0 && rot_dim % 2 == 0 && rot_dim <= head_size,
             "fk_rotary_embedding: rot_dim %d must be even and <= head_size %d", rot_dim,
             head_size);
  FK_REQUIRE(q_row_stride >= static_cast<int64_t>(num_heads) * head_size &&
                 (!key || k_row_stride >= static_cast<int64_t>(num_kv_heads) * head_size),
             "fk_rotary_embedding: row stride shorter than the heads it holds");
  FK_REQUIRE(max_position >= 0, "fk_rotary_embedding: negative max_position");
  // No cache rows: every position is out of range and leaves its token unchanged.
  if (tokens == 0 || max_position == 0) return FK_OK;
  FK_REQUIRE(positions && query && cos_sin, "fk_rotary_embedding: null pointer");
  hipStream_t s = fk::as_stream(stream);
  const bool neox = is_neox != 0;
  switch (dtype) {
    case FK_DTYPE_BF16:
      return fk::launch_t<fk::BF16>(cache_dtype, positions, query, q_row_stride, key,
                                    k_row_stride, cos_sin, max_position, tokens, num_heads,
                                    num_kv_heads, head_size, rot_dim, neox, s);
    case FK_DTYPE_F16:
      return fk::launch_t<fk::F16>(cache_dtype, positions, query, q_row_stride, key,
                                   k_row_stride, cos_sin, max_position, tokens, num_heads,
                                   num_kv_heads, head_size, rot_dim, neox, s);
    case FK_DTYPE_F32:
      return fk::launch_t<fk::F32>(cache_dtype, positions, query, q_row_stride, key,
                                   k_row_stride, cos_sin, max_position, tokens, num_heads,
                                   num_kv_heads, head_size, rot_dim, neox, s);
    default:
      return fk::set_error(FK_ERR_UNSUPPORTED, "fk_rotary_embedding: unsupported dtype %d",
                           dtype);
  }
}
