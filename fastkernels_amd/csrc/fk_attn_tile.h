// MFMA tile helpers shared by the paged attention kernels (decode and prefill).
//
// A wave processes 16 keys x 16 query columns at a time, at head size D = 64,
// 128 or 256.  Let r = lane % 16, g = lane / 16.
//   S[t, j] = K[t, :] . Q[j, :]   D / 32 x v_mfma_f32_16x16x32_bf16:
//     A = K tile (row t = r, 8 dims per lane per MFMA), B = Q^T (column j = r),
//     both with the same dim permutation, so lane (r, g) receives S[4g + i, r].
//   O[j, d] += P[j, t] V[t, d]    D / 16 x v_mfma_f32_16x16x16bf16_1k (one per
//     16-dim slice): A = P, whose layout (row j = r, tokens 4g..4g+3) is exactly
//     the S layout above, so the probabilities never leave their lane; B = V
//     (column = dim (D/16) r + slice, tokens 4g..4g+3).  A lane loads D / 16
//     contiguous dims of each of its 4 V rows and regroups them with byte
//     permutes.
// Lane (r, g) of the O accumulators holds O[column 4g + i][dims (D/16) r ..
// (D/16) r + D/16 - 1].
#pragma once

#include "fk_common.h"

namespace fk {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kTile = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// Reductions over the four 16-lane rows of a wave (lanes r, r+16, r+32, r+48)
// with the gfx950 row-swap permutes (VALU, no LDS traffic): each swap returns
// a lane's own value and its partner row's value in some order, so combining
// the two outputs symmetrically reduces each row pair.
__device__ __forceinline__ float pair_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}

// Softmax denominator of a row with running max m and sum l (log2 units) once
// an attention sink of logit sink2 (log2 units; -inf = none) joins it:
// l + 2^(sink2 - m).  A row with no visible key (l = 0) stays 0.
__device__ __forceinline__ float with_sink(float l, float m, float sink2) {
  return (l > 0.f && sink2 != kNegInf) ? l + __builtin_amdgcn_exp2f(sink2 - m) : l;
}

// Low / high 16-bit halves of a and b packed as (a, b): one v_perm_b32 each
// (byte selectors over {b, a}, a in bytes 0-3).
__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);  // (a & 0xffff) | (b << 16)
}
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);  // (a >> 16) | (b & 0xffff0000)
}

// 4 OCP e4m3fn bytes -> 4 bf16 holding float(x) * s rounded to nearest even:
// the per-tensor fp8 dequant of _cast_kv_tile (triton_unified_attention.py:
// 64-67), (data.to(float32) * scale).to(q.dtype).  With s = 1 it is exact (every
// e4m3fn value is a bf16 value).
__device__ __forceinline__ uint2 fp8x4_to_bf16x4(uint32_t w, float s) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
  const bf16x2_t a = {static_cast<__bf16>(lo[0] * s), static_cast<__bf16>(lo[1] * s)};
  const bf16x2_t b = {static_cast<__bf16>(hi[0] * s), static_cast<__bf16>(hi[1] * s)};
  return make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
}

// KV loads (plain cached loads: marking them non-temporal measured slower).
__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint2 ld8(const uint8_t* p) { return *reinterpret_cast<const uint2*>(p); }

// Value of `x` held by lane 4g + i (g = this lane's row group), for the O
// row 4g + i this lane accumulates.  Rows >= kG are padding and get lane i's.
template <int kG>
__device__ __forceinline__ float row_value(float x, int g, int i) {
  float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(x), i));
  if constexpr (kG > 4) {
    const float a1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(x), 4 + i));
    if constexpr (kG > 8) {
      const float a2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(x), 8 + i));
      const float a3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(x), 12 + i));
      a = g == 0 ? a : g == 1 ? a1 : g == 2 ? a2 : a3;
    } else {
      a = g == 1 ? a1 : a;
    }
  }
  return a;
}

// P as the A operand: row r (query column), k = keys 4g..4g+3 (RNE bf16 pack).
__device__ __forceinline__ short4_t p_operand(const float (&pr)[4]) {
  const bf16x2_t p01 = {static_cast<__bf16>(pr[0]), static_cast<__bf16>(pr[1])};
  const bf16x2_t p23 = {static_cast<__bf16>(pr[2]), static_cast<__bf16>(pr[3])};
  return __builtin_bit_cast(
      short4_t, make_uint2(__builtin_bit_cast(uint32_t, p01), __builtin_bit_cast(uint32_t, p23)));
}

// ---------------------------------------------------------------------------
// With N = D / 32 K chunks per row and D / 16 dims per lane: S = K Q^T takes N
// 16x16x32 MFMAs; lane (r, g) holds V dims (D/16) r .. (D/16) r + D/16 - 1 of
// rows 4g .. 4g+3 as NW = D / 32 words per row, and P.V takes D / 16 16x16x16
// MFMAs, slice d accumulating dim (D/16) r + d of query column 4g + i in o[d][i].
// ---------------------------------------------------------------------------
template <int N>
__device__ __forceinline__ floatx4_t qk_scores_n(const uint4 (&kc)[N], const bf16x8_t (&qb)[N]) {
  floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < N; ++c)
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kc[c]), qb[c],
                                                 acc, 0, 0, 0);
  return acc;
}

// B operands of P.V from the V rows held as words (2 bf16 dims per word): slice d
// takes dim d of rows 4g .. 4g+3.
template <int NW>
__device__ __forceinline__ void v_operands_w(const uint32_t (&vw)[4][NW], short4_t (&vb)[2 * NW]) {
#pragma unroll
  for (int d = 0; d < 2 * NW; ++d) {
    const int wi = d >> 1;
    uint32_t b01, b23;
    if (d & 1) {
      b01 = hi_pair(vw[0][wi], vw[1][wi]);
      b23 = hi_pair(vw[2][wi], vw[3][wi]);
    } else {
      b01 = lo_pair(vw[0][wi], vw[1][wi]);
      b23 = lo_pair(vw[2][wi], vw[3][wi]);
    }
    vb[d] = __builtin_bit_cast(short4_t, make_uint2(b01, b23));
  }
}

template <int N>
__device__ __forceinline__ void pv_accumulate_n(floatx4_t (&o)[N], short4_t pa,
                                                const short4_t (&vb)[N]) {
#pragma unroll
  for (int d = 0; d < N; ++d)
    o[d] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, vb[d], o[d], 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Tile registers at head size D for the kernels that run at 64, 128 and 256
// (the decode kernel, and the prefill kernel's fp8 V rows).
// ---------------------------------------------------------------------------
// Loads of N 32-bit words from p (16-, 8- or 4-byte vectors; p is aligned to
// the vector).
template <int N>
__device__ __forceinline__ void ld_words(const uint8_t* p, uint32_t (&w)[N]) {
  if constexpr (N == 1) {
    w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (N == 2) {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    w[0] = x.x;
    w[1] = x.y;
  } else {
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      const uint4 x = *reinterpret_cast<const uint4*>(p + 16 * q);
      w[4 * q] = x.x;
      w[4 * q + 1] = x.y;
      w[4 * q + 2] = x.z;
      w[4 * q + 3] = x.w;
    }
  }
}

// Raw registers one wave loads for one 16-token tile of head size D.  Lane
// (r, g): K row r -- bf16: the D/32 16-byte chunks of dims 32c + 8g .. +7;
// fp8: the D/4 bytes of dims (D/4) g .. (D/4) g + D/4 - 1 -- and V rows 4g+i,
// dims (D/16) r .. (D/16) r + D/16 - 1, as kVWords words.  load_tile only
// issues the loads; conversion and masking happen in the consumer, after the
// loads of the following tile have been issued.
template <bool kFp8, int D>
struct DTile {
  static constexpr int kKLoads = kFp8 ? D / 64 : D / 32;  // 16-byte K loads
  static constexpr int kVWords = kFp8 ? D / 64 : D / 32;  // 32-bit words per V row
  uint4 k[kKLoads];
  uint32_t v[4][kVWords];
};

// K operand chunks (bf16, dims as described at DTile) of a loaded tile; fp8
// bytes are dequantised with scale s (fp8x4_to_bf16x4).
template <bool kFp8, int D>
__device__ __forceinline__ void k_chunks_d(const DTile<kFp8, D>& t, uint4 (&kc)[D / 32],
                                           float s = 1.f) {
  if constexpr (!kFp8) {
#pragma unroll
    for (int c = 0; c < D / 32; ++c) kc[c] = t.k[c];
  } else {
    // chunk c = bytes 8c .. 8c+7 of the lane's D/4.
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
      const uint4& src = t.k[c >> 1];
      const uint32_t w0 = (c & 1) ? src.z : src.x;
      const uint32_t w1 = (c & 1) ? src.w : src.y;
      const uint2 lo = fp8x4_to_bf16x4(w0, s), hi = fp8x4_to_bf16x4(w1, s);
      kc[c] = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
  }
}

// V row i of a loaded tile as D/32 words of bf16 pairs (zero when !keep); fp8
// bytes are dequantised with scale s.
template <bool kFp8, int D>
__device__ __forceinline__ void v_words(const DTile<kFp8, D>& t, int i, bool keep,
                                        uint32_t (&w)[D / 32], float s = 1.f) {
  if constexpr (!kFp8) {
#pragma unroll
    for (int q = 0; q < D / 32; ++q) w[q] = keep ? t.v[i][q] : 0u;
  } else {
#pragma unroll
    for (int q = 0; q < D / 64; ++q) {
      const uint2 x = fp8x4_to_bf16x4(t.v[i][q], s);
      w[2 * q] = keep ? x.x : 0u;
      w[2 * q + 1] = keep ? x.y : 0u;
    }
  }
}

// P.V B operands straight from the fp8 V rows of a loaded tile: slice d takes
// dim (D/16) r + d of rows 4g .. 4g+3, each float(x) * s rounded to bf16 (the
// dequant of fp8x4_to_bf16x4).  The rounding instruction packs two rows' values
// of one dim, so the pairs come out in operand order with no byte regrouping
// (v_words + v_operands_w pack two dims of one row, then permute).  Unless
// `all`, the bytes of row i are zeroed where !keep[i] (a NaN byte becomes 0).
template <int D>
__device__ __forceinline__ void v_operands_fp8(const DTile<true, D>& t, float s, bool all,
                                               const bool (&keep)[4], short4_t (&vb)[D / 16]) {
  constexpr int NW = D / 64;  // fp8 words per row: dims 4q .. 4q + 3 in word q
  uint32_t w[4][NW];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int q = 0; q < NW; ++q) w[i][q] = t.v[i][q];
  if (!all) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < NW; ++q) w[i][q] = keep[i] ? w[i][q] : 0u;
  }
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    float f[4][4];  // [row][dim 4q + e]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(w[i][q], false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(w[i][q], true);
      f[i][0] = lo[0] * s;
      f[i][1] = lo[1] * s;
      f[i][2] = hi[0] * s;
      f[i][3] = hi[1] * s;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bf16x2_t a = {static_cast<__bf16>(f[0][e]), static_cast<__bf16>(f[1][e])};
      const bf16x2_t b = {static_cast<__bf16>(f[2][e]), static_cast<__bf16>(f[3][e])};
      vb[4 * q + e] = __builtin_bit_cast(
          short4_t, make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)));
    }
  }
}

}  // namespace fk
