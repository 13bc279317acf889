// SwiGLU activation on the fused gate/up projection rows:
//
//   out[r, j] = r( r(silu(g)) * u ),  g = gate_up[r, j], u = gate_up[r, I + j]
//   silu(g) = g / (1 + exp(-g)) in fp32, r = round to the element type
//
// the roundings of functional.silu(gate) * up in the input dtype
// (tokserve/engine/layers.py:84-91). HBM-bound single pass: 16-byte loads of
// gate and up, one 16-byte store, a grid-stride loop over (row, 8-element
// chunk); rows whose width or pointers are not 16-byte multiples take a
// scalar loop.
#include "common.hpp"

#include <algorithm>

namespace tks {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float silu(float g) { return g / (1.f + expf(-g)); }

template <typename T>
__global__ __launch_bounds__(kThreads) void silu_mul_vec_kernel(const T *__restrict__ gu, int64_t gu_rs,
                                                                T *__restrict__ out, int64_t out_rs,
                                                                int64_t rows, int64_t inter) {
  constexpr int N = Vec<T>::N;
  const int64_t chunks = inter / N;
  const int64_t total = rows * chunks;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / chunks;
    const int64_t c = (i - r * chunks) * N;
    float g[N], u[N], o[N];
    unpack<T>(ld16(gu + r * gu_rs + c), g);
    unpack<T>(ld16(gu + r * gu_rs + inter + c), u);
#pragma unroll
    for (int k = 0; k < N; ++k) o[k] = round_through<T>(silu(g[k])) * u[k];
    st16(out + r * out_rs + c, pack<T>(o));
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void silu_mul_scalar_kernel(const T *__restrict__ gu,
                                                                   int64_t gu_rs, T *__restrict__ out,
                                                                   int64_t out_rs, int64_t rows,
                                                                   int64_t inter) {
  const int64_t total = rows * inter;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / inter;
    const int64_t j = i - r * inter;
    const float g = to_float(gu[r * gu_rs + j]);
    const float u = to_float(gu[r * gu_rs + inter + j]);
    out[r * out_rs + j] = from_float<T>(round_through<T>(silu(g)) * u);
  }
}

template <typename T>
int32_t launch(const void *gate_up, int64_t gu_rs, int64_t rows, int64_t inter, void *out,
               int64_t out_rs, hipStream_t s) {
  const T *gu = static_cast<const T *>(gate_up);
  T *o = static_cast<T *>(out);
  constexpr int N = Vec<T>::N;
  const bool vec = aligned16(gate_up) && aligned16(out) && inter % N == 0 && gu_rs % N == 0 &&
                   out_rs % N == 0;
  const int64_t work = vec ? rows * (inter / N) : rows * inter;
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(256 * 8, ceil_div(work, kThreads)));
  if (vec)
    silu_mul_vec_kernel<T><<<dim3((unsigned)blocks), kThreads, 0, s>>>(gu, gu_rs, o, out_rs, rows, inter);
  else
    silu_mul_scalar_kernel<T><<<dim3((unsigned)blocks), kThreads, 0, s>>>(gu, gu_rs, o, out_rs, rows,
                                                                          inter);
  return check_launch();
}

}  // namespace
}  // namespace tks

using namespace tks;

extern "C" int32_t tks_silu_mul(const void *gate_up, int64_t gate_up_row_stride, int64_t num_rows,
                                int64_t intermediate_size, void *out, int64_t out_row_stride,
                                int32_t dtype, tks_stream_t stream) {
  if (num_rows < 0 || intermediate_size < 0) return TKS_ERR_VALUE;
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (num_rows == 0 || intermediate_size == 0) return TKS_OK;
  if (!gate_up || !out || gate_up_row_stride < 2 * intermediate_size ||
      out_row_stride < intermediate_size)
    return TKS_ERR_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TKS_FLOAT32:
      return launch<float>(gate_up, gate_up_row_stride, num_rows, intermediate_size, out,
                           out_row_stride, s);
    case TKS_FLOAT16:
      return launch<_Float16>(gate_up, gate_up_row_stride, num_rows, intermediate_size, out,
                              out_row_stride, s);
    default:
      return launch<bf16_t>(gate_up, gate_up_row_stride, num_rows, intermediate_size, out,
                            out_row_stride, s);
  }
}
