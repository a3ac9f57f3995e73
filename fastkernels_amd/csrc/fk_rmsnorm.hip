// RMSNorm and fused residual-add + RMSNorm for the decode step.
//
// Numerics follow RMSNorm.forward_native (fastkernels/tasks/baseline/L1/
// rms_norm.py:97-118):
//   s        = fp32(x) + fp32(residual)          (fused variant only)
//   residual = cast(s)
//   x_hat    = cast(s * rsqrt(mean(s^2) + eps))  (variance of the fp32 sum)
//   out      = cast(fp32(x_hat) * fp32(weight))
// where cast() rounds to the tensor dtype (round-to-nearest-even).
//
// MI355X mapping: one work-group of W wave64s per row (W = 1 up to 128
// 16-byte vectors, else 4: one wave per SIMD, so a long row's conversion and
// normalisation work is spread over the CU instead of one SIMD).  The row stays
// in VGPRs between the sum-of-squares pass and the normalise pass, so HBM
// traffic is the minimal read x, read residual, write residual, write x (the
// vLLM kernel re-reads the residual for its second pass, rms_norm.cu:
// 1370-1407).  Every access is a 16-byte vector; the row reduction is a 6-step
// wave64 butterfly, then LDS across the W waves.  Rows that do not fit the
// register-resident path use a work-group-per-row kernel that re-reads the row.
#include "fk_common.h"

namespace fk {
namespace {

// W waves per row; each lane holds VPT 16-byte vectors of the row (vector
// tid + 64 W j, j < VPT).
template <typename T, int VPT, int W, bool kFused>
__global__ __launch_bounds__(64 * W) void rmsnorm_wave_row(
    typename T::storage* out, int64_t out_row_stride,  // may alias x (fused, in place)
    typename T::storage* x, int64_t x_row_stride,
    typename T::storage* __restrict__ residual, int64_t residual_row_stride,
    const typename T::storage* __restrict__ weight, int64_t hidden, float eps) {
  using V = Vec16<T>;
  constexpr int N = V::N;
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;  // 0 .. 64 W - 1
  const int64_t nvec = hidden / N;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * x_row_stride);

  // Loads are unconditional (lanes past the row re-read its last vector and are
  // masked below): guarding each load with a branch makes the compiler wait for
  // it before issuing the next, serialising VPT memory latencies.
  float s[VPT][N];
  float ss = 0.f;
  V xv[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t vi = lane + 64 * W * j;
    xv[j].raw = xr[vi < nvec ? vi : nvec - 1];
  }
  // The weight row is needed only after the reduction; issue it now.
  const uint4* wr = reinterpret_cast<const uint4*>(weight);
  V wv[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t vi = lane + 64 * W * j;
    wv[j].raw = wr[vi < nvec ? vi : nvec - 1];
  }
  if constexpr (kFused) {
    uint4* rr = reinterpret_cast<uint4*>(residual + row * residual_row_stride);
    V rv[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int64_t vi = lane + 64 * W * j;
      rv[j].raw = rr[vi < nvec ? vi : nvec - 1];
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int64_t vi = lane + 64 * W * j;
      const bool in_row = vi < nvec;
      V nr;
#pragma unroll
      for (int e = 0; e < N; ++e) {
        s[j][e] = T::to_f32(xv[j].e[e]) + T::to_f32(rv[j].e[e]);
        nr.e[e] = T::from_f32(s[j][e]);
        ss = in_row ? sumsq_add(ss, s[j][e]) : ss;
      }
      if (in_row) rr[vi] = nr.raw;
    }
  } else {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const bool in_row = lane + 64 * W * j < nvec;
#pragma unroll
      for (int e = 0; e < N; ++e) {
        s[j][e] = T::to_f32(xv[j].e[e]);
        ss = in_row ? sumsq_add(ss, s[j][e]) : ss;
      }
    }
  }
  ss = wave_sum(ss);
  if constexpr (W > 1) {
    __shared__ float red[W];
    if ((lane & 63) == 0) red[lane >> 6] = ss;
    __syncthreads();
    ss = red[0];
#pragma unroll
    for (int w = 1; w < W; ++w) ss += red[w];
  }
  const float inv = rms_inv(ss, static_cast<float>(hidden), eps);
  uint4* orow = reinterpret_cast<uint4*>(out + row * out_row_stride);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t vi = lane + 64 * W * j;
    V ov;
#pragma unroll
    for (int e = 0; e < N; ++e) ov.e[e] = rms_apply<T>(s[j][e], inv, T::to_f32(wv[j].e[e]));
    if (vi < nvec) orow[vi] = ov.raw;
  }
}

// Work-group per row, any hidden size or alignment.  Pass 1 accumulates the
// sum of squares; pass 2 re-reads x (and residual), recomputes the fp32 sum and
// writes.  Each lane owns elements i = lane (mod 256) in both passes and reads
// an element before writing it, so the in-place fused variant (out == x) never
// reads a value another lane has already overwritten.
template <typename T, bool kFused>
__global__ __launch_bounds__(256) void rmsnorm_block_row(
    typename T::storage* out, int64_t out_row_stride,  // may alias x (fused, in place)
    typename T::storage* x, int64_t x_row_stride,
    typename T::storage* __restrict__ residual, int64_t residual_row_stride,
    const typename T::storage* __restrict__ weight, int64_t hidden, float eps) {
  const int64_t row = blockIdx.x;
  typename T::storage* xr = x + row * x_row_stride;
  typename T::storage* rr = kFused ? residual + row * residual_row_stride : nullptr;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < hidden; i += 256) {
    float v = T::to_f32(xr[i]);
    if constexpr (kFused) v += T::to_f32(rr[i]);
    ss = sumsq_add(ss, v);
  }
  __shared__ float red[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = red[0] + red[1] + red[2] + red[3];
  const float inv = rms_inv(ss, static_cast<float>(hidden), eps);
  typename T::storage* orow = out + row * out_row_stride;
  // Same element ownership as pass 1: lane i only touches elements i (mod 256).
  for (int64_t i = threadIdx.x; i < hidden; i += 256) {
    float v = T::to_f32(xr[i]);
    if constexpr (kFused) {
      v += T::to_f32(rr[i]);
      rr[i] = T::from_f32(v);
    }
    orow[i] = rms_apply<T>(v, inv, T::to_f32(weight[i]));
  }
}

template <typename T, bool kFused>
int launch_t(void* out, int64_t out_row_stride, void* x, int64_t x_row_stride, void* residual,
             int64_t residual_row_stride, const void* weight, int64_t rows, int64_t hidden,
             float eps, hipStream_t stream, const char* name) {
  using S = typename T::storage;
  constexpr int N = Vec16<T>::N;
  const int64_t es = sizeof(S);
  bool vec = (hidden % N == 0) && ((x_row_stride * es) % 16 == 0) &&
             ((out_row_stride * es) % 16 == 0) && aligned16(x) && aligned16(out) &&
             aligned16(weight);
  if (kFused) vec = vec && ((residual_row_stride * es) % 16 == 0) && aligned16(residual);
  const int64_t nvec = hidden / N;
  const dim3 grid(static_cast<unsigned>(rows));
  auto* o = static_cast<S*>(out);
  auto* xp = static_cast<S*>(x);
  auto* rp = static_cast<S*>(residual);
  const auto* wp = static_cast<const S*>(weight);
#define FK_RMS_WAVE(VPT, W)                                                                    \
  hipLaunchKernelGGL((rmsnorm_wave_row<T, VPT, W, kFused>), grid, dim3(64 * W), 0, stream, o,   \
                     out_row_stride, xp, x_row_stride, rp, residual_row_stride, wp, hidden, eps)
  if (vec && nvec <= 64) {
    FK_RMS_WAVE(1, 1);
  } else if (vec && nvec <= 128) {
    FK_RMS_WAVE(2, 1);
  } else if (vec && nvec <= 256) {
    FK_RMS_WAVE(1, 4);
  } else if (vec && nvec <= 512) {
    FK_RMS_WAVE(2, 4);
  } else if (vec && nvec <= 1024) {
    FK_RMS_WAVE(4, 4);
  } else if (vec && nvec <= 2048) {
    FK_RMS_WAVE(8, 4);
  } else if (vec && nvec <= 4096) {
    FK_RMS_WAVE(16, 4);
  } else {
    hipLaunchKernelGGL((rmsnorm_block_row<T, kFused>), grid, dim3(256), 0, stream, o,
                       out_row_stride, xp, x_row_stride, rp, residual_row_stride, wp, hidden,
                       eps);
  }
#undef FK_RMS_WAVE
  return check_launch(name);
}

template <bool kFused>
int dispatch(void* out, int64_t out_row_stride, void* x, int64_t x_row_stride, void* residual,
             int64_t residual_row_stride, const void* weight, int64_t rows, int64_t hidden,
             float eps, int dtype, void* stream, const char* name) {
  FK_REQUIRE(rows >= 0 && hidden >= 0, "%s: negative size", name);
  FK_REQUIRE(rows <= 0x7fffffffLL, "%s: too many rows (%lld)", name, (long long)rows);
  FK_REQUIRE(x_row_stride >= hidden && out_row_stride >= hidden, "%s: row stride < hidden", name);
  if (kFused) FK_REQUIRE(residual_row_stride >= hidden, "%s: residual row stride < hidden", name);
  if (rows == 0 || hidden == 0) return FK_OK;
  FK_REQUIRE(out && x && weight && (!kFused || residual), "%s: null pointer", name);
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case FK_DTYPE_BF16:
      return launch_t<BF16, kFused>(out, out_row_stride, x, x_row_stride, residual,
                                    residual_row_stride, weight, rows, hidden, eps, s, name);
    case FK_DTYPE_F16:
      return launch_t<F16, kFused>(out, out_row_stride, x, x_row_stride, residual,
                                   residual_row_stride, weight, rows, hidden, eps, s, name);
    case FK_DTYPE_F32:
      return launch_t<F32, kFused>(out, out_row_stride, x, x_row_stride, residual,
                                   residual_row_stride, weight, rows, hidden, eps, s, name);
    default:
      return set_error(FK_ERR_UNSUPPORTED, "%s: unsupported dtype %d", name, dtype);
  }
}

}  // namespace
}  // namespace fk

extern "C" int fk_rmsnorm(void* out, int64_t out_row_stride, const void* x, int64_t x_row_stride,
                          const void* weight, int64_t rows, int64_t hidden, float eps, int dtype,
                          void* stream) {
  return fk::dispatch<false>(out, out_row_stride, const_cast<void*>(x), x_row_stride, nullptr,
                             0, weight, rows, hidden, eps, dtype, stream, "fk_rmsnorm");
}

extern "C" int fk_fused_add_rmsnorm(void* x, int64_t x_row_stride, void* residual,
                                    int64_t residual_row_stride, const void* weight,
                                    int64_t rows, int64_t hidden, float eps, int dtype,
                                    void* stream) {
  return fk::dispatch<true>(x, x_row_stride, x, x_row_stride, residual, residual_row_stride,
                            weight, rows, hidden, eps, dtype, stream, "fk_fused_add_rmsnorm");
}
