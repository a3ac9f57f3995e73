// Device and host helpers shared by the gfx950 decode-step kernels.
//
// Numeric conversions are written out explicitly (round-to-nearest-even for
// fp32 -> bf16/f16, exact widening for bf16/f16/fp8 -> fp32) so that every
// kernel rounds exactly where the reference's PyTorch formulas round.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fastkernels_amd.h"

namespace fk {

// ---------------------------------------------------------------------------
// Error reporting (thread-local message behind fk_last_error()).
// ---------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Compute units of the current device (queried once per device).
int num_cus();

#define FK_REQUIRE(cond, ...)                                  \
  do {                                                         \
    if (!(cond)) return ::fk::set_error(FK_ERR_INVALID_ARG, __VA_ARGS__); \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// Scalar conversions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even fp32 -> bf16; NaN maps to the canonical quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  // The hardware conversion rounds to nearest even.  The empty asm pins f as an
  // fp32 value first: otherwise the compiler may fold the producing fma into a
  // mixed-precision fma that rounds to fp16 directly, which differs (rarely, by
  // one ulp) from rounding the fp32 result, as torch does, and differs between
  // kernels that inline the same arithmetic.
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Element-type traits: storage type + widening / narrowing.
struct BF16 {
  using storage = uint16_t;
  static constexpr int kDtype = FK_DTYPE_BF16;
  __device__ __forceinline__ static float to_f32(storage v) { return bf16_to_f32(v); }
  __device__ __forceinline__ static storage from_f32(float f) { return f32_to_bf16(f); }
  // Round an fp32 value to this type and back (models a tensor op's rounding).
  __device__ __forceinline__ static float round(float f) { return bf16_to_f32(f32_to_bf16(f)); }
};
struct F16 {
  using storage = uint16_t;
  static constexpr int kDtype = FK_DTYPE_F16;
  __device__ __forceinline__ static float to_f32(storage v) { return f16_to_f32(v); }
  __device__ __forceinline__ static storage from_f32(float f) { return f32_to_f16(f); }
  __device__ __forceinline__ static float round(float f) { return f16_to_f32(f32_to_f16(f)); }
};
struct F32 {
  using storage = float;
  static constexpr int kDtype = FK_DTYPE_F32;
  __device__ __forceinline__ static float to_f32(storage v) { return v; }
  __device__ __forceinline__ static storage from_f32(float f) { return f; }
  __device__ __forceinline__ static float round(float f) { return f; }
};

// fp32 -> OCP e4m3fn code: round to nearest even, |x| >= 448 saturates to
// +-448, NaN stays NaN (0x7F with the sign), subnormals below 2^-6.
__device__ __forceinline__ uint8_t f32_to_e4m3fn_sat(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const float a = __builtin_fabsf(x);
  if (a != a) return static_cast<uint8_t>(sign | 0x7Fu);
  if (a >= 448.f) return static_cast<uint8_t>(sign | 0x7Eu);
  if (a < 0.015625f) {  // 2^-6: subnormal grid of 2^-9 (exact scaling)
    const uint32_t m = static_cast<uint32_t>(__builtin_rintf(a * 512.f));  // 0..8; 8 = 2^-6
    return static_cast<uint8_t>(sign | m);
  }
  const int e = static_cast<int>((u >> 23) & 0xFFu) - 127;  // -6 .. 8
  const uint32_t mant = u & 0x7FFFFFu;
  uint32_t r = mant >> 20;
  const uint32_t rem = mant & 0xFFFFFu;
  r += (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) ? 1u : 0u;
  uint32_t code = (static_cast<uint32_t>(e + 7) << 3) + r;  // r == 8 carries into the exponent
  if (code > 0x7Eu) code = 0x7Eu;
  return static_cast<uint8_t>(sign | code);
}

// 16-byte vector of storage elements.
template <typename T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(typename T::storage);
  union {
    uint4 raw;
    typename T::storage e[N];
  };
};

// ---------------------------------------------------------------------------
// Arithmetic shared by the separate row ops and the fused ones, written with
// explicit fused multiply-adds so that every kernel that inlines them rounds
// identically, whatever contraction the compiler would choose at each site.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sumsq_add(float acc, float v) { return __builtin_fmaf(v, v, acc); }
// 1 / sqrt(mean + eps) for a row of n elements whose squares sum to ss.
__device__ __forceinline__ float rms_inv(float ss, float n, float eps) {
  return 1.0f / __builtin_sqrtf(ss / n + eps);
}
// cast(cast(v * inv) * w): forward_native's two rounding points.
template <typename T>
__device__ __forceinline__ typename T::storage rms_apply(float v, float inv, float w) {
  return T::from_f32(T::round(v * inv) * w);
}
// Rotation of the pair (x, y) by (c, s): x c - y s and y c + x s, one rounding.
__device__ __forceinline__ float rope_x(float x, float y, float c, float s) {
  return __builtin_fmaf(x, c, -(y * s));
}
__device__ __forceinline__ float rope_y(float x, float y, float c, float s) {
  return __builtin_fmaf(y, c, x * s);
}

// ---------------------------------------------------------------------------
// Wave64 reductions (butterfly over all 64 lanes; every lane gets the result).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

}  // namespace fk
