// RMSNorm, optionally fused with the residual add that precedes it.
//
//   x   = to_in(input + residual)            (fused path; written to residual_out)
//   out = to_out(w * to_in(x * 1/sqrt(sum(x^2)/D + eps)))
//
// Order of roundings follows RMSNorm.forward (tokserve/engine/layers.py:29-42)
// and the Triton kernel (tokserve/kernels/_triton_rmsnorm.py:30-35): fp32
// reduction, normalised value rounded to the input dtype, then one product
// with the weight. One 256-thread workgroup per row; the row stays in
// registers (one HBM read and one write per element; each thread's chunk is sized so
// the wider of its load and its store is 16 bytes, keeping every wave access one
// contiguous span).
#include "common.hpp"

namespace tks {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxChunks = 8;  // chunks per thread kept in registers

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

// E elements of T at p (16-byte aligned groups) to and from floats, as one vector
// access of E * sizeof(T) bytes (8, 16 or 32 bytes; other sizes element by element).
template <typename T, int E>
__device__ __forceinline__ void load_elems(const T *p, float *f) {
  constexpr int kBytes = E * static_cast<int>(sizeof(T));
  if constexpr (kBytes == 16) {
    unpack<T>(ld16(p), f);
  } else if constexpr (kBytes == 32) {
    unpack<T>(ld16(p), f);
    unpack<T>(ld16(p + 16 / sizeof(T)), f + 16 / sizeof(T));
  } else if constexpr (kBytes == 8) {
    const uint2 v = *reinterpret_cast<const uint2 *>(p);
    float both[16 / sizeof(T)];
    unpack<T>(make_uint4(v.x, v.y, 0u, 0u), both);
#pragma unroll
    for (int i = 0; i < E; ++i) f[i] = both[i];
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) f[i] = to_float(p[i]);
  }
}
template <typename T, int E>
__device__ __forceinline__ void store_elems(T *p, const float *f) {
  constexpr int kBytes = E * static_cast<int>(sizeof(T));
  if constexpr (kBytes == 16) {
    st16(p, pack<T>(f));
  } else if constexpr (kBytes == 32) {
    st16(p, pack<T>(f));
    st16(p + 16 / sizeof(T), pack<T>(f + 16 / sizeof(T)));
  } else if constexpr (kBytes == 8) {
    float both[16 / sizeof(T)] = {};
#pragma unroll
    for (int i = 0; i < E; ++i) both[i] = f[i];
    const uint4 v = pack<T>(both);
    *reinterpret_cast<uint2 *>(p) = make_uint2(v.x, v.y);
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) p[i] = from_float<T>(f[i]);
  }
}

// Elements per thread chunk: as many as make the widest of the input and output
// accesses 16 bytes, so every load and every store instruction of a wave covers one
// contiguous span (fp32 output of a bf16 row: 8-byte loads, 16-byte stores).
template <typename TI, typename TO>
constexpr int chunk_elems() {
  return 16 / static_cast<int>(sizeof(TI) > sizeof(TO) ? sizeof(TI) : sizeof(TO));
}

// Vector path: hidden % E == 0 and hidden <= kThreads * KC * E (KC chunks per thread).
template <typename TI, typename TW, typename TO, bool RESID, int KC>
__global__ __launch_bounds__(kThreads) void rms_norm_vec_kernel(NormArgs<TI, TW, TO> a) {
#pragma clang fp contract(off)
  constexpr int E = chunk_elems<TI, TO>();
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  const int chunks = a.hidden / E;
  float x[KC][E], w[KC][E];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = threadIdx.x + k * kThreads;
    if (c < chunks) {
      // The weight is requested with the row, not after the reduction: one memory
      // latency per row instead of two.
      load_elems<TW, E>(a.w + c * E, w[k]);
      load_elems<TI, E>(a.in + row * a.in_rs + c * E, x[k]);
      if constexpr (RESID) {
        float r[E];
        load_elems<TI, E>(a.res + row * a.res_rs + c * E, r);
#pragma unroll
        for (int j = 0; j < E; ++j) x[k][j] = round_through<TI>(x[k][j] + r[j]);
        store_elems<TI, E>(a.res_out + row * a.res_out_rs + c * E, x[k]);
      }
#pragma unroll
      for (int j = 0; j < E; ++j) ss += x[k][j] * x[k][j];
    }
  }
  const float total = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(total / static_cast<float>(a.hidden) + a.eps);
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = threadIdx.x + k * kThreads;
    if (c < chunks) {
      float y[E];
#pragma unroll
      for (int j = 0; j < E; ++j) y[j] = w[k][j] * round_through<TI>(x[k][j] * inv);
      store_elems<TO, E>(a.out + row * a.out_rs + c * E, y);
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
  constexpr int E = chunk_elems<TI, TO>();
  const bool resid = res != nullptr;
  bool vec = hidden % E == 0 && hidden <= kThreads * kMaxChunks * E && in_rs % E == 0 &&
             out_rs % E == 0 && aligned16(in) && aligned16(w) && aligned16(out);
  if (resid)
    vec = vec && res_rs % E == 0 && res_out_rs % E == 0 && aligned16(res) && aligned16(res_out);
  const dim3 grid(static_cast<unsigned>(rows));
  if (vec) {
    const int per_thread = static_cast<int>(ceil_div(hidden / E, kThreads));
#define TKS_VEC(KC)                                                                        \
  {                                                                                        \
    if (resid)                                                                             \
      rms_norm_vec_kernel<TI, TW, TO, true, KC><<<grid, kThreads, 0, s>>>(a);              \
    else                                                                                   \
      rms_norm_vec_kernel<TI, TW, TO, false, KC><<<grid, kThreads, 0, s>>>(a);             \
  }
    if (per_thread <= 1) TKS_VEC(1)
    else if (per_thread <= 2) TKS_VEC(2)
    else if (per_thread <= 4) TKS_VEC(4)
    else TKS_VEC(8)
#undef TKS_VEC
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
