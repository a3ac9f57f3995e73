// SiLU-and-mul (SwiGLU gate) for the MLP of the decode step.
//
// out[r, j] = cast(fp32(cast(silu(fp32(x[r, j])))) * fp32(x[r, d + j])),  j < d
// The activation is rounded to the dtype before the product, as in
// SiluAndMul.forward_native (fastkernels/tasks/baseline/L1/silu_and_mul.py:19-22:
// F.silu(x[..., :d]) * x[..., d:] in the tensor dtype) and in the reference's
// CUDA kernel (silu_and_mul.cu:714-738,823-830).
//
// MI355X mapping: a 2-D grid (row, column block); each lane handles one
// 16-byte vector of the gate half and the matching vector of the up half and
// writes one 16-byte output vector, so the op is three fully coalesced streams.
// Rows sit on grid.x (the dimension without the 65535 limit), and a work-group
// strides over rows by the grid width, so any token count runs in one launch.
#include "fk_common.h"

namespace fk {
namespace {

// silu(g) = g / (1 + e^-g) with the hardware reciprocal (v_rcp_f32, about 1 ulp)
// instead of an IEEE division: the activation is rounded to the 8-bit-mantissa
// dtype right after, so the two agree except at rounding ties.  g -> -inf gives
// -0 as the division does (rcp(inf) = 0); g = -inf gives NaN, as -inf / inf does.
__device__ __forceinline__ float silu_f32(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

template <typename T>
__global__ __launch_bounds__(256) void silu_and_mul_vec(typename T::storage* __restrict__ out,
                                                        int64_t out_row_stride,
                                                        const typename T::storage* __restrict__ x,
                                                        int64_t x_row_stride, int64_t rows,
                                                        int64_t d) {
  using V = Vec16<T>;
  constexpr int N = V::N;
  const int64_t vi = static_cast<int64_t>(blockIdx.y) * 256 + threadIdx.x;
  if (vi * N >= d) return;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const typename T::storage* xr = x + row * x_row_stride;
    V g, u, o;
    g.raw = *reinterpret_cast<const uint4*>(xr + vi * N);
    u.raw = *reinterpret_cast<const uint4*>(xr + d + vi * N);
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float a = T::round(silu_f32(T::to_f32(g.e[e])));
      o.e[e] = T::from_f32(a * T::to_f32(u.e[e]));
    }
    *reinterpret_cast<uint4*>(out + row * out_row_stride + vi * N) = o.raw;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void silu_and_mul_scalar(
    typename T::storage* __restrict__ out, int64_t out_row_stride,
    const typename T::storage* __restrict__ x, int64_t x_row_stride, int64_t rows, int64_t d) {
  const int64_t j = static_cast<int64_t>(blockIdx.y) * 256 + threadIdx.x;
  if (j >= d) return;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const typename T::storage* xr = x + row * x_row_stride;
    const float a = T::round(silu_f32(T::to_f32(xr[j])));
    out[row * out_row_stride + j] = T::from_f32(a * T::to_f32(xr[d + j]));
  }
}

template <typename T>
int launch_t(void* out, int64_t out_row_stride, const void* x, int64_t x_row_stride,
             int64_t rows, int64_t d, hipStream_t stream) {
  using S = typename T::storage;
  constexpr int N = Vec16<T>::N;
  const int64_t es = sizeof(S);
  const bool vec = d % N == 0 && (x_row_stride * es) % 16 == 0 &&
                   (out_row_stride * es) % 16 == 0 && aligned16(x) && aligned16(out);
  const int64_t per = vec ? d / N : d;
  const int64_t col_blocks = (per + 255) / 256;
  FK_REQUIRE(col_blocks <= 65535, "fk_silu_and_mul: d %lld too wide (at most %lld)",
             (long long)d, (long long)(65535LL * 256 * (vec ? N : 1)));
  // 256-lane work-groups: grid.x * 256 must fit in 32 bits; beyond kMaxRowGroups
  // rows each work-group takes several rows.
  constexpr int64_t kMaxRowGroups = int64_t(1) << 22;
  const dim3 grid(static_cast<unsigned>(rows < kMaxRowGroups ? rows : kMaxRowGroups),
                  static_cast<unsigned>(col_blocks));
  if (vec)
    hipLaunchKernelGGL(silu_and_mul_vec<T>, grid, dim3(256), 0, stream, static_cast<S*>(out),
                       out_row_stride, static_cast<const S*>(x), x_row_stride, rows, d);
  else
    hipLaunchKernelGGL(silu_and_mul_scalar<T>, grid, dim3(256), 0, stream,
                       static_cast<S*>(out), out_row_stride, static_cast<const S*>(x),
                       x_row_stride, rows, d);
  return check_launch("fk_silu_and_mul");
}

}  // namespace
}  // namespace fk

extern "C" int fk_silu_and_mul(void* out, int64_t out_row_stride, const void* x,
                               int64_t x_row_stride, int64_t rows, int64_t d, int dtype,
                               void* stream) {
  FK_REQUIRE(rows >= 0 && d >= 0, "fk_silu_and_mul: negative size");
  FK_REQUIRE(x_row_stride >= 2 * d && out_row_stride >= d,
             "fk_silu_and_mul: row stride shorter than the row");
  if (rows == 0 || d == 0) return FK_OK;
  FK_REQUIRE(out && x, "fk_silu_and_mul: null pointer");
  hipStream_t s = fk::as_stream(stream);
  switch (dtype) {
    case FK_DTYPE_BF16:
      return fk::launch_t<fk::BF16>(out, out_row_stride, x, x_row_stride, rows, d, s);
    case FK_DTYPE_F16:
      return fk::launch_t<fk::F16>(out, out_row_stride, x, x_row_stride, rows, d, s);
    case FK_DTYPE_F32:
      return fk::launch_t<fk::F32>(out, out_row_stride, x, x_row_stride, rows, d, s);
    default:
      return fk::set_error(FK_ERR_UNSUPPORTED, "fk_silu_and_mul: unsupported dtype %d", dtype);
  }
}
