// Elementwise addition of two 1-D vectors (vector_add,
// tokserve/kernels/vector.py:6-41 and _triton_vector.py:11-25).
//
// HBM-bound: 16-byte loads and stores where all three pointers are 16-byte
// aligned, a scalar loop otherwise; a grid-stride loop over at most 8 waves per
// CU of workgroups. fp16 sums are formed in fp32 and rounded to fp16; that
// double rounding gives the correctly rounded half-precision sum because fp32
// carries 24 >= 2 * 11 + 2 significand bits (Figueroa's double-rounding bound
// for +, -, *, /).
#include "common.hpp"

#include <algorithm>

namespace tks {
namespace {

constexpr int kThreads = 256;

template <typename T>
__global__ __launch_bounds__(kThreads) void vector_add_vec_kernel(const T *__restrict__ x,
                                                                  const T *__restrict__ y,
                                                                  T *__restrict__ out, int64_t n_vec) {
  constexpr int N = Vec<T>::N;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n_vec; i += stride) {
    float a[N], b[N];
    unpack<T>(ld16(x + i * N), a);
    unpack<T>(ld16(y + i * N), b);
#pragma unroll
    for (int k = 0; k < N; ++k) a[k] += b[k];
    st16(out + i * N, pack<T>(a));
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void vector_add_scalar_kernel(const T *__restrict__ x,
                                                                     const T *__restrict__ y,
                                                                     T *__restrict__ out,
                                                                     int64_t begin, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
    out[i] = from_float<T>(to_float(x[i]) + to_float(y[i]));
}

template <typename T>
int32_t launch(const void *x, const void *y, void *out, int64_t n, hipStream_t s) {
  const T *xt = static_cast<const T *>(x);
  const T *yt = static_cast<const T *>(y);
  T *ot = static_cast<T *>(out);
  constexpr int N = Vec<T>::N;
  const int64_t max_blocks = 256 * 8;
  int64_t done = 0;
  if (aligned16(x) && aligned16(y) && aligned16(out) && n >= N) {
    const int64_t n_vec = n / N;
    const int64_t blocks = std::min<int64_t>(max_blocks, ceil_div(n_vec, kThreads));
    vector_add_vec_kernel<T><<<dim3((unsigned)blocks), kThreads, 0, s>>>(xt, yt, ot, n_vec);
    done = n_vec * N;
  }
  if (done < n) {
    const int64_t blocks = std::min<int64_t>(max_blocks, ceil_div(n - done, kThreads));
    vector_add_scalar_kernel<T><<<dim3((unsigned)blocks), kThreads, 0, s>>>(xt, yt, ot, done, n);
  }
  return check_launch();
}

}  // namespace
}  // namespace tks

using namespace tks;

extern "C" int32_t tks_vector_add(const void *x, const void *y, void *out, int64_t num_elements,
                                  int32_t dtype, tks_stream_t stream) {
  if (num_elements < 0) return TKS_ERR_VALUE;
  if (dtype != TKS_FLOAT32 && dtype != TKS_FLOAT16) return TKS_ERR_TYPE;
  if (num_elements == 0) return TKS_OK;
  if (!x || !y || !out) return TKS_ERR_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == TKS_FLOAT32 ? launch<float>(x, y, out, num_elements, s)
                              : launch<_Float16>(x, y, out, num_elements, s);
}
