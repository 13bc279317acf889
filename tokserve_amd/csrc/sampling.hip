// Greedy token selection on a (rows, vocab) logits batch.
//
// torch.argmax semantics (select_greedy, tokserve/generation/greedy.py:18):
// the first index of the maximum; NaN compares greater than every number and
// the first NaN wins. One 256-thread workgroup per row, one pass over HBM.
#include "common.hpp"

namespace tks {
namespace {

constexpr int kThreads = 256;

// True if candidate (v, i) beats the incumbent (bv, bi).
__device__ __forceinline__ bool beats(float v, int64_t i, float bv, int64_t bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void argmax_kernel(const T *__restrict__ logits,
                                                          int64_t row_stride, int64_t vocab,
                                                          int64_t *__restrict__ out) {
  __shared__ float sv[kThreads];
  __shared__ int64_t si[kThreads];
  const T *row = logits + blockIdx.x * row_stride;
  float best = -INFINITY;
  int64_t bi = vocab;  // sentinel index larger than any real one
  for (int64_t i = threadIdx.x; i < vocab; i += kThreads) {
    const float v = to_float(row[i]);
    if (beats(v, i, best, bi)) {
      best = v;
      bi = i;
    }
  }
  sv[threadIdx.x] = best;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) {
      const float v = sv[threadIdx.x + w];
      const int64_t i = si[threadIdx.x + w];
      if (beats(v, i, sv[threadIdx.x], si[threadIdx.x])) {
        sv[threadIdx.x] = v;
        si[threadIdx.x] = i;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[blockIdx.x] = si[0] < vocab ? si[0] : 0;
}

}  // namespace
}  // namespace tks

using namespace tks;

extern "C" int32_t tks_argmax(const void *logits, int64_t row_stride, int64_t num_rows,
                              int64_t vocab_size, int64_t *out_ids, int32_t dtype,
                              tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (num_rows < 0 || vocab_size <= 0 || num_rows > 0x7fffffff) return TKS_ERR_VALUE;
  if (num_rows == 0) return TKS_OK;
  if (!logits || !out_ids) return TKS_ERR_VALUE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(num_rows));
  switch (dtype) {
    case TKS_FLOAT32:
      argmax_kernel<float><<<grid, kThreads, 0, s>>>(static_cast<const float *>(logits),
                                                     row_stride, vocab_size, out_ids);
      break;
    case TKS_FLOAT16:
      argmax_kernel<_Float16><<<grid, kThreads, 0, s>>>(static_cast<const _Float16 *>(logits),
                                                        row_stride, vocab_size, out_ids);
      break;
    default:
      argmax_kernel<bf16_t><<<grid, kThreads, 0, s>>>(static_cast<const bf16_t *>(logits),
                                                      row_stride, vocab_size, out_ids);
      break;
  }
  return check_launch();
}
