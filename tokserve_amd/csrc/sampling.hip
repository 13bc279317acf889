// Greedy token selection on a (rows, vocab) logits batch.
//
// torch.argmax semantics (select_greedy, tokserve/generation/greedy.py:18):
// the first index of the maximum; NaN compares greater than every number and
// the first NaN wins. One 512-thread workgroup per row, one pass over HBM. Rows
// whose start and stride are 16-byte multiples are read in 16-byte chunks, up to
// kUnroll per thread issued before the first is compared (a 32,000-entry bf16
// row is one batch of loads); other rows take the element-by-element loop.
#include "common.hpp"

namespace tks {
namespace {

constexpr int kThreads = 512;

// True if candidate (v, i) beats the incumbent (bv, bi).
__device__ __forceinline__ bool beats(float v, int64_t i, float bv, int64_t bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

// The workgroup's best (value, index) pair, from each thread's, into out: across
// each wave by lane swaps, then the waves' winners through LDS.
__device__ __forceinline__ void block_best(float best, int64_t bi, int64_t vocab, int64_t *out) {
  int idx = static_cast<int>(bi);  // indices are below 2^31 (vocab is checked)
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float v = __shfl_xor(best, off, 64);
    const int i = __shfl_xor(idx, off, 64);
    if (beats(v, i, best, idx)) {
      best = v;
      idx = i;
    }
  }
  __shared__ float sv[kThreads / 64];
  __shared__ int si[kThreads / 64];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = best;
    si[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kThreads / 64; ++w)
      if (beats(sv[w], si[w], best, idx)) {
        best = sv[w];
        idx = si[w];
      }
    *out = idx < vocab ? idx : 0;
  }
}

// A thread meets its entries in increasing index order, so within a thread the
// first maximum is kept by a strict comparison (and the first NaN by taking a NaN
// only over a number).
__device__ __forceinline__ void take_if_better(float v, int64_t i, float &best, int64_t &bi) {
  if (v > best || (v != v && best == best)) {
    best = v;
    bi = i;
  }
}

constexpr int kUnroll = 16;

template <typename T>
__global__ __launch_bounds__(kThreads) void argmax_vec_kernel(const T *__restrict__ logits,
                                                              int64_t row_stride, int64_t vocab,
                                                              int64_t *__restrict__ out) {
  constexpr int N = Vec<T>::N;
  const T *row = logits + blockIdx.x * row_stride;
  const int64_t chunks = vocab / N;
  float best = -INFINITY;
  int64_t bi = vocab;  // sentinel index larger than any real one
  for (int64_t c0 = threadIdx.x; c0 < chunks; c0 += (int64_t)kThreads * kUnroll) {
    uint4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t c = c0 + (int64_t)u * kThreads;
      v[u] = c < chunks ? ld16(row + c * N) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t c = c0 + (int64_t)u * kThreads;
      if (c < chunks) {
        float f[N];
        unpack<T>(v[u], f);
#pragma unroll
        for (int k = 0; k < N; ++k) take_if_better(f[k], c * N + k, best, bi);
      }
    }
  }
  for (int64_t i = chunks * N + threadIdx.x; i < vocab; i += kThreads)
    take_if_better(to_float(row[i]), i, best, bi);
  block_best(best, bi, vocab, out + blockIdx.x);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void argmax_kernel(const T *__restrict__ logits,
                                                          int64_t row_stride, int64_t vocab,
                                                          int64_t *__restrict__ out) {
  const T *row = logits + blockIdx.x * row_stride;
  float best = -INFINITY;
  int64_t bi = vocab;  // sentinel index larger than any real one
  for (int64_t i = threadIdx.x; i < vocab; i += kThreads) take_if_better(to_float(row[i]), i, best, bi);
  block_best(best, bi, vocab, out + blockIdx.x);
}

template <typename T>
void launch_argmax(const void *logits, int64_t row_stride, int64_t num_rows, int64_t vocab,
                   int64_t *out, hipStream_t s) {
  const T *x = static_cast<const T *>(logits);
  const dim3 grid(static_cast<unsigned>(num_rows));
  if (aligned16(logits) && (row_stride * static_cast<int64_t>(sizeof(T))) % 16 == 0)
    argmax_vec_kernel<T><<<grid, kThreads, 0, s>>>(x, row_stride, vocab, out);
  else
    argmax_kernel<T><<<grid, kThreads, 0, s>>>(x, row_stride, vocab, out);
}

}  // namespace
}  // namespace tks

using namespace tks;

extern "C" int32_t tks_argmax(const void *logits, int64_t row_stride, int64_t num_rows,
                              int64_t vocab_size, int64_t *out_ids, int32_t dtype,
                              tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (num_rows < 0 || vocab_size <= 0 || num_rows > 0x7fffffff || vocab_size > 0x7fffffff)
    return TKS_ERR_VALUE;
  if (num_rows == 0) return TKS_OK;
  if (!logits || !out_ids) return TKS_ERR_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TKS_FLOAT32: launch_argmax<float>(logits, row_stride, num_rows, vocab_size, out_ids, s); break;
    case TKS_FLOAT16: launch_argmax<_Float16>(logits, row_stride, num_rows, vocab_size, out_ids, s); break;
    default: launch_argmax<bf16_t>(logits, row_stride, num_rows, vocab_size, out_ids, s); break;
  }
  return check_launch();
}
