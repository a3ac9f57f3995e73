// Fused per-head q/k RMSNorm + rotary embedding + KV-cache store: the part of
// the attention block between the qkv projection and the decode attention.
//
// Reference order (fastkernels/tasks/baseline/L2/attention.py:120-140, then
// attention_impl.py:313-325):
//   q = q_norm(q.view(N, Hq, D)), k = k_norm(k.view(N, Hk, D))   (Qwen3; optional)
//   q, k = rotary_emb(positions, q, k)                          (rotary_emb.py)
//   store_kvcache(k, v, k_cache, v_cache, slot_mapping)         (store_kvcache.py)
// The per-head norm is RMSNorm.forward_native (rms_norm.py:97-118) on rows of
// D: cast(cast(x rsqrt(mean x^2 + eps)) w).  The rotation is the one of
// fk_rotary.hip (cos/sin rounded to the dtype, products formed in fp32 and
// rounded once); tokens whose position is outside [0, max_position) are not
// rotated, as there.  All arithmetic goes through the helpers the separate
// RMSNorm and rotary kernels use, in the same element order, so the result is
// bit-identical to running those ops and store_kvcache one after another.
//
// MI355X mapping: one work-group per token.  A head row (D elements) is held
// by D/8 lanes (bf16; D/4 for fp32), one 16-byte vector per lane: the row's
// sum of squares is a butterfly inside the lane group, and the NeoX partner
// half-row comes from the lane rot/2/8 positions away by a cross-lane read.
// q and k heads are rewritten in place in their (strided) rows, k and v heads
// are written to the cache slot, so a token's q, k and v are read once and
// written once instead of three times over three launches.
#include "fk_common.h"

namespace fk {
namespace {

struct QkParams {
  const int64_t* positions;
  void* query;
  int64_t q_row_stride;
  void* key;
  int64_t k_row_stride;
  const void* value;
  int64_t v_row_stride;
  const void* q_weight;  // [D] or null (no norm)
  const void* k_weight;
  float eps;
  const void* cos_sin;
  int64_t max_position;
  int rot_dim;
  void* k_cache;
  void* v_cache;
  const void* slot_mapping;
  int slot_is_i64;
  int64_t num_slots;
  int num_heads, num_kv_heads, head_size;
};

// kLanes lanes per head row (D / N, a power of two <= 64).  kNorm: apply the
// per-head RMSNorm to q and k before rotating.
template <typename T, typename CT, bool kNeox, int kLanes, bool kNorm>
__global__ __launch_bounds__(256) void qk_norm_rope_store_kernel(QkParams P) {
  using S = typename T::storage;
  using CS = typename CT::storage;
  using V = Vec16<T>;
  constexpr int N = V::N;
  constexpr int kGroups = 256 / kLanes;
  const int64_t tok = blockIdx.x;
  const int sub = threadIdx.x % kLanes;
  const int grp = threadIdx.x / kLanes;
  const int64_t pos = P.positions[tok];
  const bool rotate = pos >= 0 && pos < P.max_position;
  const int64_t slot = P.slot_is_i64 ? static_cast<const int64_t*>(P.slot_mapping)[tok]
                                     : static_cast<const int32_t*>(P.slot_mapping)[tok];
  const bool store = slot >= 0 && slot < P.num_slots;
  const int hq = P.num_heads, hk = P.num_kv_heads, D = P.head_size;
  const int half = P.rot_dim / 2;
  const int64_t cache_row = static_cast<int64_t>(hk) * D;
  const CS* cs = static_cast<const CS*>(P.cos_sin) + (rotate ? pos : 0) * P.rot_dim;
  const int e0 = sub * N;  // first element of this lane's vector in the head row
  // Rows of the 16 lanes of a group are processed in lock step; every lane of
  // the wave runs the same trip count, so the cross-lane reads below always
  // have their partner lanes active.  Up to kBatch trips' row loads (and the
  // norm weights) are issued before any of them is processed: the stores of one
  // trip would otherwise keep the next trip's loads (same qkv buffer, unknown
  // aliasing to the compiler) behind them, one memory round trip per trip.
  constexpr int kBatch = 4;
  const int units = hq + 2 * hk;
  const int trips = (units + kGroups - 1) / kGroups;
  V wq, wk;
  if constexpr (kNorm) {
    wq.raw = *reinterpret_cast<const uint4*>(static_cast<const S*>(P.q_weight) + e0);
    wk.raw = *reinterpret_cast<const uint4*>(static_cast<const S*>(P.k_weight) + e0);
  }
  for (int t0 = 0; t0 < trips; t0 += kBatch) {
    V xb[kBatch];
    S* rows[kBatch];
    int heads[kBatch];
    bool lives[kBatch], qs[kBatch], vs[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int u = grp + (t0 + b) * kGroups;
      lives[b] = t0 + b < trips && u < units;
      const int uu = (t0 + b < trips && u < units) ? u : units - 1;  // dead slots re-read the last row
      qs[b] = uu < hq;
      vs[b] = uu >= hq + hk;
      heads[b] = qs[b] ? uu : (vs[b] ? uu - hq - hk : uu - hq);
      if (qs[b])
        rows[b] = static_cast<S*>(P.query) + tok * P.q_row_stride + static_cast<int64_t>(heads[b]) * D;
      else if (vs[b])
        rows[b] = const_cast<S*>(static_cast<const S*>(P.value)) + tok * P.v_row_stride +
                  static_cast<int64_t>(heads[b]) * D;
      else
        rows[b] = static_cast<S*>(P.key) + tok * P.k_row_stride + static_cast<int64_t>(heads[b]) * D;
      xb[b].raw = *reinterpret_cast<const uint4*>(rows[b] + e0);
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      if (t0 + b >= trips) break;  // uniform over the work-group
      const bool live = lives[b], is_q = qs[b], is_v = vs[b];
      const int head = heads[b];
      S* row = rows[b];
      V x = xb[b];
      if (!is_v) {  // uniform over the lane group
        if constexpr (kNorm) {
          const V& w = is_q ? wq : wk;
          float ss = 0.f;
#pragma unroll
          for (int e = 0; e < N; ++e) ss = sumsq_add(ss, T::to_f32(x.e[e]));
#pragma unroll
          for (int off = kLanes / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
          const float inv = rms_inv(ss, static_cast<float>(D), P.eps);
#pragma unroll
          for (int e = 0; e < N; ++e) x.e[e] = rms_apply<T>(T::to_f32(x.e[e]), inv, T::to_f32(w.e[e]));
        }
        if constexpr (kNeox) {
          // Lane vectors of the first half pair with those half/N lanes later.
          const int hv = half / N;
          const bool first = sub < hv;
          const bool in_rot = sub < 2 * hv;
          const int src = static_cast<int>(threadIdx.x & 63) + (first ? hv : (in_rot ? -hv : 0));
          V y;
          y.raw.x = __shfl(x.raw.x, src, 64);
          y.raw.y = __shfl(x.raw.y, src, 64);
          y.raw.z = __shfl(x.raw.z, src, 64);
          y.raw.w = __shfl(x.raw.w, src, 64);
          if (rotate && in_rot) {
            const int i0 = first ? e0 : e0 - half;  // cos/sin index of element 0
#pragma unroll
            for (int e = 0; e < N; ++e) {
              const float c = T::round(CT::to_f32(cs[i0 + e]));
              const float sn = T::round(CT::to_f32(cs[half + i0 + e]));
              const float mine = T::to_f32(x.e[e]);
              const float other = T::to_f32(y.e[e]);
              x.e[e] = first ? T::from_f32(rope_x(mine, other, c, sn))
                             : T::from_f32(rope_y(other, mine, c, sn));
            }
          }
        } else {
          if (rotate && e0 < P.rot_dim) {
#pragma unroll
            for (int j = 0; j < N / 2; ++j) {
              const int i = e0 / 2 + j;
              const float c = T::round(CT::to_f32(cs[i]));
              const float sn = T::round(CT::to_f32(cs[half + i]));
              const float a = T::to_f32(x.e[2 * j]);
              const float bb = T::to_f32(x.e[2 * j + 1]);
              x.e[2 * j] = T::from_f32(rope_x(a, bb, c, sn));
              x.e[2 * j + 1] = T::from_f32(rope_y(a, bb, c, sn));
            }
          }
        }
        if (live) *reinterpret_cast<uint4*>(row + e0) = x.raw;
      }
      if (live && !is_q && store) {
        S* dst = static_cast<S*>(is_v ? P.v_cache : P.k_cache) + slot * cache_row +
                 static_cast<int64_t>(head) * D + e0;
        *reinterpret_cast<uint4*>(dst) = x.raw;
      }
    }
  }
}

template <typename T, typename CT, bool kNeox, bool kNorm>
int launch_lanes(const QkParams& P, int64_t tokens, hipStream_t stream) {
  constexpr int N = Vec16<T>::N;
  const dim3 grid(static_cast<unsigned>(tokens));
#define FK_QK(L)                                                                        \
  hipLaunchKernelGGL((qk_norm_rope_store_kernel<T, CT, kNeox, L, kNorm>), grid, dim3(256), \
                     0, stream, P)
  switch (P.head_size / N) {
    case 4: FK_QK(4); break;
    case 8: FK_QK(8); break;
    case 16: FK_QK(16); break;
    case 32: FK_QK(32); break;
    case 64: FK_QK(64); break;
    default:
      return set_error(FK_ERR_UNSUPPORTED,
                       "fk_qk_norm_rope_store: head_size %d must be 4..64 16-byte vectors "
                       "(a power of two)", P.head_size);
  }
#undef FK_QK
  return check_launch("fk_qk_norm_rope_store");
}

template <typename T, typename CT>
int launch_tc(const QkParams& P, bool neox, int64_t tokens, hipStream_t stream) {
  const bool norm = P.q_weight != nullptr;
  if (neox)
    return norm ? launch_lanes<T, CT, true, true>(P, tokens, stream)
                : launch_lanes<T, CT, true, false>(P, tokens, stream);
  return norm ? launch_lanes<T, CT, false, true>(P, tokens, stream)
              : launch_lanes<T, CT, false, false>(P, tokens, stream);
}

template <typename T>
int launch_t(const QkParams& P, int cache_dtype, bool neox, int64_t tokens, hipStream_t stream) {
  using S = typename T::storage;
  constexpr int N = Vec16<T>::N;
  const int64_t es = sizeof(S);
  const bool ok = P.head_size % N == 0 && (neox ? (P.rot_dim / 2) % N == 0 : P.rot_dim % N == 0) &&
                  (P.q_row_stride * es) % 16 == 0 && (P.k_row_stride * es) % 16 == 0 &&
                  (P.v_row_stride * es) % 16 == 0 && aligned16(P.query) && aligned16(P.key) &&
                  aligned16(P.value) && aligned16(P.k_cache) && aligned16(P.v_cache) &&
                  (P.q_weight == nullptr || (aligned16(P.q_weight) && aligned16(P.k_weight)));
  if (!ok)
    return set_error(FK_ERR_UNSUPPORTED,
                     "fk_qk_norm_rope_store: needs 16-byte aligned rows, caches and weights, "
                     "and rot_dim/2 (NeoX) or rot_dim (GPT-J) a multiple of %d", N);
  if (cache_dtype == FK_DTYPE_F32) return launch_tc<T, F32>(P, neox, tokens, stream);
  if (cache_dtype == T::kDtype) return launch_tc<T, T>(P, neox, tokens, stream);
  return set_error(FK_ERR_UNSUPPORTED,
                   "fk_qk_norm_rope_store: cos_sin dtype %d must be f32 or the query dtype %d",
                   cache_dtype, T::kDtype);
}

}  // namespace
}  // namespace fk

extern "C" int fk_qk_norm_rope_store(
    const int64_t* positions, void* query, int64_t q_row_stride, void* key,
    int64_t k_row_stride, const void* value, int64_t v_row_stride, const void* q_weight,
    const void* k_weight, float eps, const void* cos_sin, int cache_dtype, int64_t max_position,
    int rot_dim, int is_neox, void* k_cache, void* v_cache, const void* slot_mapping,
    int slot_is_i64, int64_t num_slots, int64_t tokens, int num_heads, int num_kv_heads,
    int head_size, int dtype, void* stream) {
  const char* name = "fk_qk_norm_rope_store";
  FK_REQUIRE(tokens >= 0 && tokens <= 0x7fffffffLL && num_slots >= 0,
             "%s: bad token or slot count", name);
  FK_REQUIRE(num_heads > 0 && num_kv_heads > 0 && head_size > 0,
             "%s: bad head counts (heads=%d kv_heads=%d head_size=%d)", name, num_heads,
             num_kv_heads, head_size);
  FK_REQUIRE(rot_dim > 0 && rot_dim % 2 == 0 && rot_dim <= head_size,
             "%s: rot_dim %d must be even and <= head_size %d", name, rot_dim, head_size);
  FK_REQUIRE((q_weight == nullptr) == (k_weight == nullptr),
             "%s: pass both q and k norm weights or neither", name);
  FK_REQUIRE(q_row_stride >= static_cast<int64_t>(num_heads) * head_size &&
                 k_row_stride >= static_cast<int64_t>(num_kv_heads) * head_size &&
                 v_row_stride >= static_cast<int64_t>(num_kv_heads) * head_size,
             "%s: row stride shorter than the heads it holds", name);
  if (tokens == 0) return FK_OK;
  FK_REQUIRE(positions && query && key && value && cos_sin && k_cache && v_cache &&
                 slot_mapping,
             "%s: null pointer", name);
  fk::QkParams P{positions, query, q_row_stride, key, k_row_stride, value, v_row_stride,
                 q_weight, k_weight, eps, cos_sin, max_position, rot_dim, k_cache, v_cache,
                 slot_mapping, slot_is_i64 ? 1 : 0, num_slots, num_heads, num_kv_heads,
                 head_size};
  hipStream_t s = fk::as_stream(stream);
  const bool neox = is_neox != 0;
  switch (dtype) {
    case FK_DTYPE_BF16: return fk::launch_t<fk::BF16>(P, cache_dtype, neox, tokens, s);
    case FK_DTYPE_F16: return fk::launch_t<fk::F16>(P, cache_dtype, neox, tokens, s);
    case FK_DTYPE_F32: return fk::launch_t<fk::F32>(P, cache_dtype, neox, tokens, s);
    default: return fk::set_error(FK_ERR_UNSUPPORTED, "%s: unsupported dtype %d", name, dtype);
  }
}
