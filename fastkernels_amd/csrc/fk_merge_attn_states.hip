// merge_attn_states: log-sum-exp merge of two partial attention results.
//
// For token t, head h (lse tensors are [H, T], natural log; out / prefix /
// suffix are [T, H, D] with a head stride and a token stride):
//   p, s  = prefix_lse[h, t], suffix_lse[h, t], with +inf read as -inf
//   M     = max(p, s); ep = e^(p - M); es = e^(s - M); E = ep + es
//   out   = prefix * (ep / E) + suffix * (es / E)   (fp32, rounded once)
//   out_lse[h, t] = log(E) + M
// When M = -inf (no keys on either side) the prefix rows are copied and
// out_lse = -inf.  Tokens t >= prefill_tokens_with_context copy the suffix
// rows and lse.  Every infinite lse is read as -inf.
// fp8 output (output_scale, the USE_FP8_OUTPUT form of merge_attn_states.cu:
// 2436-2571): every output value -- the fp32 merge, or the copied prefix /
// suffix value -- is multiplied by 1 / output_scale (the reciprocal formed once in
// fp32), clamped to [-448, 448] with fmin / fmax (so NaN becomes 448) and
// rounded to the nearest e4m3fn value.
// This is merge_attn_states of fastkernels/tasks/baseline/L1/merge_attn_states.py:
// 30-100 (vLLM's kernel; Triton form in triton_merge_attn_states.py), section
// 2.2 of arXiv 2501.01005.
//
// MI355X mapping: a group of head_size/8 (bf16) or head_size/4 (fp32) lanes per
// (token, head), each lane moving 16-byte vectors with the two lse values
// broadcast, so the op is three coalesced streams plus the lse reads.
#include "fk_common.h"

namespace fk {
namespace {

struct MergeParams {
  void* out;
  int64_t out_token_stride, out_head_stride;
  float* out_lse;
  const void* prefix;
  const void* suffix;
  int64_t in_token_stride, in_head_stride;
  const float* prefix_lse;
  const float* suffix_lse;
  int64_t tokens;
  int heads, head_size;
  int64_t prefill_tokens;  // tokens >= this copy the suffix
  const float* output_scale;  // fp8 output: device fp32 scalar
};

// fp8 output code of value v with the reciprocal scale inv.
__device__ __forceinline__ uint8_t fp8_out(float v, float inv) {
  return f32_to_e4m3fn_sat(fmaxf(-448.f, fminf(v * inv, 448.f)));
}
// N output codes packed little-endian (N = 4 or 8 bytes).
template <int N>
struct Fp8Pack;
template <>
struct Fp8Pack<4> {
  using type = uint32_t;
};
template <>
struct Fp8Pack<8> {
  using type = uint2;
};

// Weights of one (token, head) from its prefix and suffix lse (p, s), computed
// without branches so that the row and lse loads all issue before any wait.
//   copy_suffix: a token without a prefix (t >= prefill_tokens): the suffix row
//                and lse are copied;
//   copy_prefix: both lse -inf (no keys on either side): the prefix row, which is
//                then the empty result, is copied with lse -inf;
//   otherwise    out = prefix * ps + suffix * ss, lse = log(E) + M.
// Copies move the bits, so inf/nan rows stay as they are.
struct MergeWeights {
  float ps, ss, lse;
  bool copy_prefix, copy_suffix;
};

__device__ __forceinline__ MergeWeights merge_weights(float p, float s, bool tail) {
  const float inf = __builtin_huge_valf();
  const float s_raw = s;
  p = (p == inf || p == -inf) ? -inf : p;
  s = (s == inf || s == -inf) ? -inf : s;
  const float m = fmaxf(p, s);
  const bool empty = m == -inf;
  const float ms = empty ? 0.f : m;
  const float ep = expf(p - ms);
  const float es = expf(s - ms);
  const float e = ep + es;
  MergeWeights w;
  w.ps = ep / e;
  w.ss = es / e;
  w.copy_suffix = tail;
  w.copy_prefix = !tail && empty;
  w.lse = tail ? s_raw : (empty ? -inf : logf(e) + m);
  return w;
}

__device__ __forceinline__ uint32_t pick(const MergeWeights& w, uint32_t merged, uint32_t a,
                                         uint32_t b) {
  return w.copy_suffix ? b : (w.copy_prefix ? a : merged);
}

// Vector path: kLanes lanes (a power of two <= 64) share one (token, head) and
// move 16-byte vectors, so a 128-wide bf16 head is 16 lanes and a wave covers
// four heads: every lane carries data.  With kLoop false (rows of at most
// kLanes vectors) each lane moves one vector: its row loads (clamped into the
// row) and the two lse loads all issue before the first wait, so a head costs
// one memory round trip.  kLoop strides longer rows 64 vectors at a time.
template <typename T, int kLanes, bool kLoop, bool kFp8Out>
__global__ __launch_bounds__(256) void merge_attn_states_vec(MergeParams P) {
  using S = typename T::storage;
  using V = Vec16<T>;
  constexpr int N = V::N;
  const float inv = kFp8Out ? 1.f / *P.output_scale : 1.f;
  const uint32_t total = static_cast<uint32_t>(P.tokens * P.heads);
  const uint32_t unit = blockIdx.x * (256 / kLanes) + threadIdx.x / kLanes;
  if (unit >= total) return;
  const int sub = threadIdx.x % kLanes;
  const uint32_t heads = static_cast<uint32_t>(P.heads);
  const uint32_t tt = unit / heads;
  const uint32_t h = unit - tt * heads;
  const int64_t t = tt;
  const S* pin = static_cast<const S*>(P.prefix) + t * P.in_token_stride + h * P.in_head_stride;
  const S* sin = static_cast<const S*>(P.suffix) + t * P.in_token_stride + h * P.in_head_stride;
  S* o = static_cast<S*>(P.out) + t * P.out_token_stride + h * P.out_head_stride;
  uint8_t* o8 = static_cast<uint8_t*>(P.out) + t * P.out_token_stride + h * P.out_head_stride;
  const int64_t lse_idx = static_cast<int64_t>(h) * P.tokens + t;
  const int i0 = kLoop ? sub * N : min(sub * N, P.head_size - N);
  V a, b;
  a.raw = *reinterpret_cast<const uint4*>(pin + i0);
  b.raw = *reinterpret_cast<const uint4*>(sin + i0);
  const float pl = P.prefix_lse[lse_idx];
  const float sl = P.suffix_lse[lse_idx];
  const MergeWeights w = merge_weights(pl, sl, t >= P.prefill_tokens);
  if (sub == 0 && P.out_lse) P.out_lse[lse_idx] = w.lse;
  for (int i = sub * N; i < P.head_size; i += kLanes * N) {
    if (kLoop && i != i0) {
      a.raw = *reinterpret_cast<const uint4*>(pin + i);
      b.raw = *reinterpret_cast<const uint4*>(sin + i);
    }
    if constexpr (kFp8Out) {
      uint8_t c[N];
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float fa = T::to_f32(a.e[e]), fb = T::to_f32(b.e[e]);
        c[e] = fp8_out(w.copy_suffix ? fb : (w.copy_prefix ? fa : fa * w.ps + fb * w.ss), inv);
      }
      typename Fp8Pack<N>::type packed;
      __builtin_memcpy(&packed, c, N);
      *reinterpret_cast<typename Fp8Pack<N>::type*>(o8 + i) = packed;
      if (!kLoop) break;
      continue;
    }
    V r;
#pragma unroll
    for (int e = 0; e < N; ++e)
      r.e[e] = T::from_f32(T::to_f32(a.e[e]) * w.ps + T::to_f32(b.e[e]) * w.ss);
    uint4 res;
    res.x = pick(w, r.raw.x, a.raw.x, b.raw.x);
    res.y = pick(w, r.raw.y, a.raw.y, b.raw.y);
    res.z = pick(w, r.raw.z, a.raw.z, b.raw.z);
    res.w = pick(w, r.raw.w, a.raw.w, b.raw.w);
    *reinterpret_cast<uint4*>(o + i) = res;
    if (!kLoop) break;
  }
}

// Scalar path (any head size / alignment): one wave per (token, head).
template <typename T, bool kFp8Out>
__global__ __launch_bounds__(256) void merge_attn_states_scalar(MergeParams P) {
  using S = typename T::storage;
  const float inv = kFp8Out ? 1.f / *P.output_scale : 1.f;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (unit >= P.tokens * P.heads) return;
  const int lane = threadIdx.x & 63;
  const int64_t t = unit / P.heads;
  const int h = static_cast<int>(unit - t * P.heads);
  const S* pin = static_cast<const S*>(P.prefix) + t * P.in_token_stride + h * P.in_head_stride;
  const S* sin = static_cast<const S*>(P.suffix) + t * P.in_token_stride + h * P.in_head_stride;
  S* o = static_cast<S*>(P.out) + t * P.out_token_stride + h * P.out_head_stride;
  const int64_t lse_idx = static_cast<int64_t>(h) * P.tokens + t;
  const MergeWeights w =
      merge_weights(P.prefix_lse[lse_idx], P.suffix_lse[lse_idx], t >= P.prefill_tokens);
  if (lane == 0 && P.out_lse) P.out_lse[lse_idx] = w.lse;
  for (int i = lane; i < P.head_size; i += 64) {
    const S a = pin[i], b = sin[i];
    if constexpr (kFp8Out) {
      const float fa = T::to_f32(a), fb = T::to_f32(b);
      static_cast<uint8_t*>(P.out)[t * P.out_token_stride + h * P.out_head_stride + i] =
          fp8_out(w.copy_suffix ? fb : (w.copy_prefix ? fa : fa * w.ps + fb * w.ss), inv);
    } else {
      o[i] = w.copy_suffix
                 ? b
                 : (w.copy_prefix ? a : T::from_f32(T::to_f32(a) * w.ps + T::to_f32(b) * w.ss));
    }
  }
}

template <typename T, int kLanes, bool kFp8Out, bool kLoop = false>
int launch_vec(const MergeParams& P, hipStream_t stream) {
  constexpr int kUnitsPerBlock = 256 / kLanes;
  const int64_t blocks = (P.tokens * P.heads + kUnitsPerBlock - 1) / kUnitsPerBlock;
  hipLaunchKernelGGL((merge_attn_states_vec<T, kLanes, kLoop, kFp8Out>),
                     dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, P);
  return check_launch("fk_merge_attn_states");
}

// kFp8Out: output elements are e4m3fn bytes (out strides in bytes), N per vector.
template <typename T, bool kFp8Out = false>
int launch_t(const MergeParams& P, hipStream_t stream) {
  constexpr int N = Vec16<T>::N;
  const int64_t es = sizeof(typename T::storage);
  const int64_t out_vec = kFp8Out ? N : 16;  // bytes of output per vector
  const int64_t oes = kFp8Out ? 1 : es;
  const bool vec = P.head_size % N == 0 && (P.in_head_stride * es) % 16 == 0 &&
                   (P.in_token_stride * es) % 16 == 0 &&
                   (P.out_head_stride * oes) % out_vec == 0 &&
                   (P.out_token_stride * oes) % out_vec == 0 &&
                   (reinterpret_cast<uintptr_t>(P.out) % out_vec) == 0 &&
                   aligned16(P.prefix) && aligned16(P.suffix);
  if (vec) {
    const int chunks = P.head_size / N;  // 16-byte vectors per head row
    if (chunks <= 1) return launch_vec<T, 1, kFp8Out>(P, stream);
    if (chunks <= 2) return launch_vec<T, 2, kFp8Out>(P, stream);
    if (chunks <= 4) return launch_vec<T, 4, kFp8Out>(P, stream);
    if (chunks <= 8) return launch_vec<T, 8, kFp8Out>(P, stream);
    if (chunks <= 16) return launch_vec<T, 16, kFp8Out>(P, stream);
    if (chunks <= 32) return launch_vec<T, 32, kFp8Out>(P, stream);
    if (chunks <= 64) return launch_vec<T, 64, kFp8Out>(P, stream);
    return launch_vec<T, 64, kFp8Out, true>(P, stream);
  }
  const int64_t units = P.tokens * P.heads;
  hipLaunchKernelGGL((merge_attn_states_scalar<T, kFp8Out>),
                     dim3(static_cast<unsigned>((units + 3) / 4)), dim3(256), 0, stream, P);
  return check_launch("fk_merge_attn_states");
}

}  // namespace
}  // namespace fk

extern "C" int fk_merge_attn_states(void* out, int64_t out_token_stride, int64_t out_head_stride,
                                    float* out_lse, const void* prefix, const float* prefix_lse,
                                    const void* suffix, const float* suffix_lse,
                                    int64_t in_token_stride, int64_t in_head_stride,
                                    int64_t tokens, int heads, int head_size,
                                    int64_t prefill_tokens_with_context, int dtype,
                                    int out_dtype, const float* output_scale, void* stream) {
  FK_REQUIRE(tokens >= 0 && heads >= 0 && head_size >= 0, "fk_merge_attn_states: negative size");
  FK_REQUIRE(tokens * heads <= 0x7fffffffLL, "fk_merge_attn_states: too many (token, head)");
  FK_REQUIRE(in_head_stride >= head_size && out_head_stride >= head_size &&
                 in_token_stride >= static_cast<int64_t>(heads) * in_head_stride &&
                 out_token_stride >= static_cast<int64_t>(heads) * out_head_stride,
             "fk_merge_attn_states: strides shorter than the rows they hold");
  if (tokens == 0 || heads == 0 || head_size == 0) return FK_OK;
  FK_REQUIRE(out && prefix && suffix && prefix_lse && suffix_lse,
             "fk_merge_attn_states: null pointer");
  FK_REQUIRE(out_dtype == dtype || out_dtype == FK_DTYPE_FP8_E4M3FN,
             "fk_merge_attn_states: out_dtype %d must be the input dtype or fp8 e4m3fn",
             out_dtype);
  const bool fp8_out = out_dtype == FK_DTYPE_FP8_E4M3FN && dtype != FK_DTYPE_FP8_E4M3FN;
  FK_REQUIRE(!fp8_out || output_scale,
             "fk_merge_attn_states: an fp8 output needs output_scale");
  fk::MergeParams P{out, out_token_stride, out_head_stride, out_lse, prefix, suffix,
                    in_token_stride, in_head_stride, prefix_lse, suffix_lse, tokens, heads,
                    head_size, prefill_tokens_with_context < 0 ? tokens
                                                               : prefill_tokens_with_context,
                    output_scale};
  hipStream_t s = fk::as_stream(stream);
  if (fp8_out) {
    switch (dtype) {
      case FK_DTYPE_BF16: return fk::launch_t<fk::BF16, true>(P, s);
      case FK_DTYPE_F16: return fk::launch_t<fk::F16, true>(P, s);
      case FK_DTYPE_F32: return fk::launch_t<fk::F32, true>(P, s);
      default: break;
    }
  }
  switch (dtype) {
    case FK_DTYPE_BF16: return fk::launch_t<fk::BF16>(P, s);
    case FK_DTYPE_F16: return fk::launch_t<fk::F16>(P, s);
    case FK_DTYPE_F32: return fk::launch_t<fk::F32>(P, s);
    default:
      return fk::set_error(FK_ERR_UNSUPPORTED, "fk_merge_attn_states: unsupported dtype %d",
                           dtype);
  }
}
