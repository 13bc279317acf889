// RMSNorm, optionally fused with the residual add that precedes it.
//
//   x   = to_in(input + residual)            (fused path; written to residual_out)
//   out = to_out(w * to_in(x * 1/sqrt(sum(x^2)/D + eps)))
//
// Order of roundings follows RMSNorm.forward (tokserve/engine/layers.py:29-42)
// and the Triton kernel (tokserve/kernels/_triton_rmsnorm.py:30-35): fp32
// reduction, normalised value rounded to the input dtype, then one product
// with the weight. One 256-thread workgroup per row; the row stays in
// registers (16-byte loads, one HBM read and one write per element).
#include "common.hpp"

namespace tks {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxChunks = 4;  // 16-byte chunks per thread kept in registers

template <typename TI, typename TW, typename TO>
struct NormArgs {
  const TI *in;
  int64_t in_rs;
  const TI *res;
  int64_t res_rs;
  TI *res_out;
  int64_t res_out_rs;
  const TW *w;
  TO *out;
  int64_t out_rs;
  int32_t hidden;
  float eps;
};

__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) t += red[i];
  return t;
}

// Loads VI elements of type T starting at p into floats (VI * sizeof(T) == 16 or VI == 1).
template <typename T, int N>
__device__ __forceinline__ void load_n(const T *p, float *f) {
  if constexpr (N * sizeof(T) == 16) {
    unpack<T>(ld16(p), f);
  } else if constexpr (N * sizeof(T) == 32) {
    unpack<T>(ld16(p), f);
    unpack<T>(ld16(p + 16 / sizeof(T)), f + 16 / sizeof(T));
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) f[i] = to_float(p[i]);
  }
}
template <typename T, int N>
__device__ __forceinline__ void store_n(T *p, const float *f) {
  if constexpr (N * sizeof(T) == 16) {
    st16(p, pack<T>(f));
  } else if constexpr (N * sizeof(T) == 32) {
    st16(p, pack<T>(f));
    st16(p + 16 / sizeof(T), pack<T>(f + 16 / sizeof(T)));
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = from_float<T>(f[i]);
  }
}

// Vector path: hidden % (16 / sizeof(TI)) == 0 and hidden <= kThreads * kMaxChunks * V.
template <typename TI, typename TW, typename TO, bool RESID>
__global__ __launch_bounds__(kThreads) void rms_norm_vec_kernel(NormArgs<TI, TW, TO> a) {
#pragma clang fp contract(off)
  constexpr int V = Vec<TI>::N;
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  const int chunks = a.hidden / V;
  float x[kMaxChunks][V];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxChunks; ++k) {
    const int c = threadIdx.x + k * kThreads;
    if (c < chunks) {
      load_n<TI, V>(a.in + row * a.in_rs + c * V, x[k]);
      if constexpr (RESID) {
        float r[V];
        load_n<TI, V>(a.res + row * a.res_rs + c * V, r);
#pragma unroll
        for (int j = 0; j < V; ++j) x[k][j] = round_through<TI>(x[k][j] + r[j]);
        store_n<TI, V>(a.res_out + row * a.res_out_rs + c * V, x[k]);
      }
#pragma unroll
      for (int j = 0; j < V; ++j) ss += x[k][j] * x[k][j];
    }
  }
  const float total = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(total / static_cast<float>(a.hidden) + a.eps);
#pragma unroll
  for (int k = 0; k < kMaxChunks; ++k) {
    const int c = threadIdx.x + k * kThreads;
    if (c < chunks) {
      float w[V], y[V];
      load_n<TW, V>(a.w + c * V, w);
#pragma unroll
      for (int j = 0; j < V; ++j) y[j] = w[j] * round_through<TI>(x[k][j] * inv);
      store_n<TO, V>(a.out + row * a.out_rs + c * V, y);
    }
  }
}

// Any hidden size: two passes over the row (the second hits in cache).
template <typename TI, typename TW, typename TO, bool RESID>
__global__ __launch_bounds__(kThreads) void rms_norm_any_kernel(NormArgs<TI, TW, TO> a) {
#pragma clang fp contract(off)
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  float ss = 0.f;
  for (int i = threadIdx.x; i < a.hidden; i += kThreads) {
    float x = to_float(a.in[row * a.in_rs + i]);
    if constexpr (RESID) x = round_through<TI>(x + to_float(a.res[row * a.res_rs + i]));
    ss += x * x;
  }
  const float total = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(total / static_cast<float>(a.hidden) + a.eps);
  for (int i = threadIdx.x; i < a.hidden; i += kThreads) {
    float x = to_float(a.in[row * a.in_rs + i]);
    if constexpr (RESID) {
      x = round_through<TI>(x + to_float(a.res[row * a.res_rs + i]));
      a.res_out[row * a.res_out_rs + i] = from_float<TI>(x);
    }
    a.out[row * a.out_rs + i] =
        from_float<TO>(to_float(a.w[i]) * round_through<TI>(x * inv));
  }
}

template <typename TI, typename TW, typename TO>
int32_t launch(const void *in, int64_t in_rs, const void *res, int64_t res_rs, void *res_out,
               int64_t res_out_rs, const void *w, void *out, int64_t out_rs, int64_t rows,
               int32_t hidden, float eps, hipStream_t s) {
  NormArgs<TI, TW, TO> a{static_cast<const TI *>(in), in_rs, static_cast<const TI *>(res),
                         res_rs, static_cast<TI *>(res_out), res_out_rs,
                         static_cast<const TW *>(w), static_cast<TO *>(out), out_rs, hidden,
                         eps};
  constexpr int V = Vec<TI>::N;
  // The weight and output are accessed V elements at a time too.
  constexpr bool wo_vec_ok = (V * sizeof(TW)) % 16 == 0 && (V * sizeof(TO)) % 16 == 0;
  const bool resid = res != nullptr;
  bool vec = wo_vec_ok && hidden % V == 0 && hidden <= kThreads * kMaxChunks * V &&
             in_rs % V == 0 && out_rs % V == 0 && aligned16(in) && aligned16(w) &&
             aligned16(out);
  if (resid)
    vec = vec && res_rs % V == 0 && res_out_rs % V == 0 && aligned16(res) && aligned16(res_out);
  const dim3 grid(static_cast<unsigned>(rows));
  if (vec) {
    if (resid)
      rms_norm_vec_kernel<TI, TW, TO, true><<<grid, kThreads, 0, s>>>(a);
    else
      rms_norm_vec_kernel<TI, TW, TO, false><<<grid, kThreads, 0, s>>>(a);
  } else {
    if (resid)
      rms_norm_any_kernel<TI, TW, TO, true><<<grid, kThreads, 0, s>>>(a);
    else
      rms_norm_any_kernel<TI, TW, TO, false><<<grid, kThreads, 0, s>>>(a);
  }
  return check_launch();
}

}  // namespace
}  // namespace tks

using namespace tks;

extern "C" int32_t tks_rms_norm(const void *input, int64_t input_row_stride, const void *residual,
                                int64_t residual_row_stride, void *residual_out,
                                int64_t residual_out_row_stride, const void *weight, void *out,
                                int64_t out_row_stride, int64_t num_rows, int32_t hidden_size,
                                float epsilon, int32_t input_dtype, int32_t weight_dtype,
                                int32_t out_dtype, tks_stream_t stream) {
  if (!valid_dtype(input_dtype) || !valid_dtype(weight_dtype) || !valid_dtype(out_dtype))
    return TKS_ERR_TYPE;
  // Torch promotion of weight * input-dtype value: fp32 weight -> fp32 out,
  // weight of the input dtype -> out in the input dtype.
  const bool promo_ok = (weight_dtype == TKS_FLOAT32 && out_dtype == TKS_FLOAT32) ||
                        (weight_dtype == input_dtype && out_dtype == input_dtype);
  if (!promo_ok) return TKS_ERR_TYPE;
  if (num_rows < 0 || hidden_size <= 0 || !(epsilon > 0.f)) return TKS_ERR_VALUE;
  if (num_rows == 0) return TKS_OK;
  if (num_rows > 0x7fffffff) return TKS_ERR_VALUE;
  if (!input || !weight || !out) return TKS_ERR_VALUE;
  if ((residual == nullptr) != (residual_out == nullptr)) return TKS_ERR_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define TKS_NORM(TI, TW, TO)                                                                  \
  return launch<TI, TW, TO>(input, input_row_stride, residual, residual_row_stride,          \
                            residual_out, residual_out_row_stride, weight, out, out_row_stride, \
                            num_rows, hidden_size, epsilon, s)
  if (weight_dtype == TKS_FLOAT32) {
    switch (input_dtype) {
      case TKS_FLOAT32: TKS_NORM(float, float, float);
      case TKS_FLOAT16: TKS_NORM(_Float16, float, float);
      default: TKS_NORM(bf16_t, float, float);
    }
  }
  if (input_dtype == TKS_FLOAT16) TKS_NORM(_Float16, _Float16, _Float16);
  TKS_NORM(bf16_t, bf16_t, bf16_t);
#undef TKS_NORM
}
