// KV append (slot_mapping scatter into paged blocks) and block-table gather.
//
// Both are pure copies, bound by HBM bandwidth: one lane moves one 16-byte
// chunk of one (token, head) row, so a wave touches 1 KiB of contiguous K (or
// V) per instruction. Pool layout [L, NB, Hkv, BS, Dh]
// (tokserve/engine/paged/storage.py:40-56); slot -> (slot / BS, slot % BS)
// (tokserve/engine/paged/block_table.py:53-67).
#include "common.hpp"

namespace tks {
namespace {

struct PoolGeom {
  int64_t layer_stride;  // NB * Hkv * BS * Dh
  int64_t block_stride;  // Hkv * BS * Dh
  int64_t head_stride;   // BS * Dh
  int64_t num_slots;     // NB * BS
  int32_t block_size;
  int32_t head_dim;
  int32_t num_kv_heads;
};

// VEC elements of type T per lane (VEC == 16 / sizeof(T) on the vector path, 1 otherwise).
template <typename T, int VEC>
__device__ __forceinline__ void copy_chunk(const T *src, T *dst) {
  if constexpr (VEC * sizeof(T) == 16) {
    st16(dst, ld16(src));
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) dst[i] = src[i];
  }
}

template <typename T, int VEC>
__global__ __launch_bounds__(256) void kv_append_kernel(
    const T *__restrict__ key, int64_t k_ts, int64_t k_hs, const T *__restrict__ value,
    int64_t v_ts, int64_t v_hs, int64_t num_tokens, T *__restrict__ key_cache,
    T *__restrict__ value_cache, PoolGeom g, int64_t layer_base,
    const int64_t *__restrict__ slot_mapping) {
  const int chunks = g.head_dim / VEC;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t per_token = static_cast<int64_t>(g.num_kv_heads) * chunks;
  if (item >= num_tokens * per_token) return;
  const int64_t t = item / per_token;
  const int rem = static_cast<int>(item - t * per_token);
  const int h = rem / chunks;
  const int d = (rem - h * chunks) * VEC;
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= g.num_slots) return;
  const int64_t block = slot / g.block_size;
  const int64_t offset = slot - block * g.block_size;
  const int64_t dst =
      layer_base + block * g.block_stride + h * g.head_stride + offset * g.head_dim + d;
  copy_chunk<T, VEC>(key + t * k_ts + h * k_hs + d, key_cache + dst);
  copy_chunk<T, VEC>(value + t * v_ts + h * v_hs + d, value_cache + dst);
}

template <typename T, int VEC>
__global__ __launch_bounds__(256) void paged_gather_kernel(
    const T *__restrict__ key_cache, const T *__restrict__ value_cache, PoolGeom g,
    int64_t layer_base, int64_t num_blocks, const int32_t *__restrict__ block_tables,
    int32_t bt_stride, const int32_t *__restrict__ seq_lens,
    const int32_t *__restrict__ cu_seqlens, int32_t max_seq_len, T *__restrict__ key_out,
    T *__restrict__ value_out, int64_t o_ts, int64_t o_hs) {
  const int b = blockIdx.y;
  const int chunks = g.head_dim / VEC;
  const int64_t per_token = static_cast<int64_t>(g.num_kv_heads) * chunks;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t p = item / per_token;
  if (p >= max_seq_len || p >= seq_lens[b]) return;
  const int rem = static_cast<int>(item - p * per_token);
  const int h = rem / chunks;
  const int d = (rem - h * chunks) * VEC;
  const int64_t block = block_tables[static_cast<int64_t>(b) * bt_stride + p / g.block_size];
  if (block < 0 || block >= num_blocks) return;
  const int64_t offset = p % g.block_size;
  const int64_t src =
      layer_base + block * g.block_stride + h * g.head_stride + offset * g.head_dim + d;
  const int64_t dst = (cu_seqlens[b] + p) * o_ts + h * o_hs + d;
  copy_chunk<T, VEC>(key_cache + src, key_out + dst);
  copy_chunk<T, VEC>(value_cache + src, value_out + dst);
}

PoolGeom make_geom(int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
                   int32_t head_dim) {
  PoolGeom g;
  g.head_stride = static_cast<int64_t>(block_size) * head_dim;
  g.block_stride = g.head_stride * num_kv_heads;
  g.layer_stride = g.block_stride * num_blocks;
  g.num_slots = num_blocks * block_size;
  g.block_size = block_size;
  g.head_dim = head_dim;
  g.num_kv_heads = num_kv_heads;
  return g;
}

bool pool_args_ok(int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
                  int32_t block_size, int32_t head_dim) {
  return num_layers > 0 && num_blocks > 0 && num_kv_heads > 0 && block_size > 0 && head_dim > 0;
}

template <typename T>
int32_t launch_append(const void *key, int64_t k_ts, int64_t k_hs, const void *value,
                      int64_t v_ts, int64_t v_hs, int64_t num_tokens, void *key_cache,
                      void *value_cache, const PoolGeom &g, int64_t layer_base,
                      const int64_t *slots, hipStream_t stream) {
  constexpr int V = Vec<T>::N;
  const bool vec = g.head_dim % V == 0 && k_ts % V == 0 && k_hs % V == 0 && v_ts % V == 0 &&
                   v_hs % V == 0 && aligned16(key) && aligned16(value) &&
                   aligned16(key_cache) && aligned16(value_cache);
  const int v = vec ? V : 1;
  const int64_t items = num_tokens * g.num_kv_heads * (g.head_dim / v);
  const dim3 grid(static_cast<unsigned>(ceil_div(items, 256)));
  if (vec)
    kv_append_kernel<T, V><<<grid, 256, 0, stream>>>(
        static_cast<const T *>(key), k_ts, k_hs, static_cast<const T *>(value), v_ts, v_hs,
        num_tokens, static_cast<T *>(key_cache), static_cast<T *>(value_cache), g, layer_base,
        slots);
  else
    kv_append_kernel<T, 1><<<grid, 256, 0, stream>>>(
        static_cast<const T *>(key), k_ts, k_hs, static_cast<const T *>(value), v_ts, v_hs,
        num_tokens, static_cast<T *>(key_cache), static_cast<T *>(value_cache), g, layer_base,
        slots);
  return check_launch();
}

template <typename T>
int32_t launch_gather(const void *key_cache, const void *value_cache, const PoolGeom &g,
                      int64_t layer_base, int64_t num_blocks, const int32_t *bt,
                      int32_t bt_stride, const int32_t *seq_lens, const int32_t *cu,
                      int32_t num_seqs, int32_t max_seq_len, void *key_out, void *value_out,
                      int64_t o_ts, int64_t o_hs, hipStream_t stream) {
  constexpr int V = Vec<T>::N;
  const bool vec = g.head_dim % V == 0 && o_ts % V == 0 && o_hs % V == 0 &&
                   aligned16(key_cache) && aligned16(value_cache) && aligned16(key_out) &&
                   aligned16(value_out);
  const int v = vec ? V : 1;
  const int64_t items = static_cast<int64_t>(max_seq_len) * g.num_kv_heads * (g.head_dim / v);
  const dim3 grid(static_cast<unsigned>(ceil_div(items, 256)), num_seqs);
  if (vec)
    paged_gather_kernel<T, V><<<grid, 256, 0, stream>>>(
        static_cast<const T *>(key_cache), static_cast<const T *>(value_cache), g, layer_base,
        num_blocks, bt, bt_stride, seq_lens, cu, max_seq_len, static_cast<T *>(key_out),
        static_cast<T *>(value_out), o_ts, o_hs);
  else
    paged_gather_kernel<T, 1><<<grid, 256, 0, stream>>>(
        static_cast<const T *>(key_cache), static_cast<const T *>(value_cache), g, layer_base,
        num_blocks, bt, bt_stride, seq_lens, cu, max_seq_len, static_cast<T *>(key_out),
        static_cast<T *>(value_out), o_ts, o_hs);
  return check_launch();
}

// ------------------------------------------------------------ fp8 pools ---
//
// E elements per lane: 16 (one 16-byte pool chunk) when rows allow it, else 1.
// Encoding divides by the pool scale in fp32 and rounds once to e4m3 after the
// clamp to +-448; decoding multiplies the exact f32 value by the scale and
// rounds once to T.

template <typename T, int E>
__device__ __forceinline__ void quantize_chunk(const T *src, uint8_t *dst, float scale) {
  float x[E];
  if constexpr (E == 16) {
    constexpr int N = Vec<T>::N;
#pragma unroll
    for (int i = 0; i < E; i += N) unpack<T>(ld16(src + i), x + i);
  } else {
    x[0] = to_float(src[0]);
  }
  encode_e4m3<E>(x, scale, dst);
}

// float(code) * scale rounded to fp32, then to T.
template <typename T, int E>
__device__ __forceinline__ void dequantize_chunk(const uint8_t *src, T *dst, float scale) {
  float f[E];
  if constexpr (E == 16) {
    unpack<fp8e4m3_t>(ld16(src), f);
  } else {
    f[0] = to_float(fp8e4m3_t{src[0]});
  }
#pragma unroll
  for (int i = 0; i < E; ++i) f[i] = fp32_value(f[i] * scale);
  if constexpr (E == 16) {
    constexpr int N = Vec<T>::N;
#pragma unroll
    for (int i = 0; i < E; i += N) st16(dst + i, pack<T>(f + i));
  } else {
    dst[0] = from_float<T>(f[0]);
  }
}

template <typename T, int E>
__global__ __launch_bounds__(256) void kv_append_fp8_kernel(
    const T *__restrict__ key, int64_t k_ts, int64_t k_hs, const T *__restrict__ value,
    int64_t v_ts, int64_t v_hs, int64_t num_tokens, uint8_t *__restrict__ key_cache,
    uint8_t *__restrict__ value_cache, PoolGeom g, int64_t layer_base,
    const int64_t *__restrict__ slot_mapping, float k_scale, float v_scale) {
  const int chunks = g.head_dim / E;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t per_token = static_cast<int64_t>(g.num_kv_heads) * chunks;
  if (item >= num_tokens * per_token) return;
  const int64_t t = item / per_token;
  const int rem = static_cast<int>(item - t * per_token);
  const int h = rem / chunks;
  const int d = (rem - h * chunks) * E;
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= g.num_slots) return;
  const int64_t block = slot / g.block_size;
  const int64_t offset = slot - block * g.block_size;
  const int64_t dst =
      layer_base + block * g.block_stride + h * g.head_stride + offset * g.head_dim + d;
  quantize_chunk<T, E>(key + t * k_ts + h * k_hs + d, key_cache + dst, k_scale);
  quantize_chunk<T, E>(value + t * v_ts + h * v_hs + d, value_cache + dst, v_scale);
}

template <typename T, int E>
__global__ __launch_bounds__(256) void paged_gather_fp8_kernel(
    const uint8_t *__restrict__ key_cache, const uint8_t *__restrict__ value_cache, PoolGeom g,
    int64_t layer_base, int64_t num_blocks, const int32_t *__restrict__ block_tables,
    int32_t bt_stride, const int32_t *__restrict__ seq_lens,
    const int32_t *__restrict__ cu_seqlens, int32_t max_seq_len, T *__restrict__ key_out,
    T *__restrict__ value_out, int64_t o_ts, int64_t o_hs, float k_scale, float v_scale) {
  const int b = blockIdx.y;
  const int chunks = g.head_dim / E;
  const int64_t per_token = static_cast<int64_t>(g.num_kv_heads) * chunks;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t p = item / per_token;
  if (p >= max_seq_len || p >= seq_lens[b]) return;
  const int rem = static_cast<int>(item - p * per_token);
  const int h = rem / chunks;
  const int d = (rem - h * chunks) * E;
  const int64_t block = block_tables[static_cast<int64_t>(b) * bt_stride + p / g.block_size];
  if (block < 0 || block >= num_blocks) return;
  const int64_t offset = p % g.block_size;
  const int64_t src =
      layer_base + block * g.block_stride + h * g.head_stride + offset * g.head_dim + d;
  const int64_t dst = (cu_seqlens[b] + p) * o_ts + h * o_hs + d;
  dequantize_chunk<T, E>(key_cache + src, key_out + dst, k_scale);
  dequantize_chunk<T, E>(value_cache + src, value_out + dst, v_scale);
}

template <typename T>
int32_t launch_append_fp8(const void *key, int64_t k_ts, int64_t k_hs, const void *value,
                          int64_t v_ts, int64_t v_hs, int64_t num_tokens, void *key_cache,
                          void *value_cache, const PoolGeom &g, int64_t layer_base,
                          const int64_t *slots, float k_scale, float v_scale,
                          hipStream_t stream) {
  constexpr int N = Vec<T>::N;
  const bool vec = g.head_dim % 16 == 0 && k_ts % N == 0 && k_hs % N == 0 && v_ts % N == 0 &&
                   v_hs % N == 0 && aligned16(key) && aligned16(value) &&
                   aligned16(key_cache) && aligned16(value_cache);
  const int e = vec ? 16 : 1;
  const int64_t items = num_tokens * g.num_kv_heads * (g.head_dim / e);
  const dim3 grid(static_cast<unsigned>(ceil_div(items, 256)));
  const T *k = static_cast<const T *>(key);
  const T *v = static_cast<const T *>(value);
  uint8_t *kc = static_cast<uint8_t *>(key_cache);
  uint8_t *vc = static_cast<uint8_t *>(value_cache);
  if (vec)
    kv_append_fp8_kernel<T, 16><<<grid, 256, 0, stream>>>(k, k_ts, k_hs, v, v_ts, v_hs,
                                                          num_tokens, kc, vc, g, layer_base,
                                                          slots, k_scale, v_scale);
  else
    kv_append_fp8_kernel<T, 1><<<grid, 256, 0, stream>>>(k, k_ts, k_hs, v, v_ts, v_hs,
                                                         num_tokens, kc, vc, g, layer_base,
                                                         slots, k_scale, v_scale);
  return check_launch();
}

template <typename T>
int32_t launch_gather_fp8(const void *key_cache, const void *value_cache, const PoolGeom &g,
                          int64_t layer_base, int64_t num_blocks, const int32_t *bt,
                          int32_t bt_stride, const int32_t *seq_lens, const int32_t *cu,
                          int32_t num_seqs, int32_t max_seq_len, void *key_out, void *value_out,
                          int64_t o_ts, int64_t o_hs, float k_scale, float v_scale,
                          hipStream_t stream) {
  constexpr int N = Vec<T>::N;
  const bool vec = g.head_dim % 16 == 0 && o_ts % N == 0 && o_hs % N == 0 &&
                   aligned16(key_cache) && aligned16(value_cache) && aligned16(key_out) &&
                   aligned16(value_out);
  const int e = vec ? 16 : 1;
  const int64_t items = static_cast<int64_t>(max_seq_len) * g.num_kv_heads * (g.head_dim / e);
  const dim3 grid(static_cast<unsigned>(ceil_div(items, 256)), num_seqs);
  const uint8_t *kc = static_cast<const uint8_t *>(key_cache);
  const uint8_t *vc = static_cast<const uint8_t *>(value_cache);
  if (vec)
    paged_gather_fp8_kernel<T, 16><<<grid, 256, 0, stream>>>(
        kc, vc, g, layer_base, num_blocks, bt, bt_stride, seq_lens, cu, max_seq_len,
        static_cast<T *>(key_out), static_cast<T *>(value_out), o_ts, o_hs, k_scale, v_scale);
  else
    paged_gather_fp8_kernel<T, 1><<<grid, 256, 0, stream>>>(
        kc, vc, g, layer_base, num_blocks, bt, bt_stride, seq_lens, cu, max_seq_len,
        static_cast<T *>(key_out), static_cast<T *>(value_out), o_ts, o_hs, k_scale, v_scale);
  return check_launch();
}

}  // namespace
}  // namespace tks

using namespace tks;

extern "C" int32_t tks_kv_append(const void *key, int64_t key_token_stride,
                                 int64_t key_head_stride, const void *value,
                                 int64_t value_token_stride, int64_t value_head_stride,
                                 int64_t num_tokens, void *key_cache, void *value_cache,
                                 int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
                                 int32_t block_size, int32_t head_dim, int32_t layer_index,
                                 const int64_t *slot_mapping, int32_t dtype,
                                 tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (!pool_args_ok(num_layers, num_blocks, num_kv_heads, block_size, head_dim) ||
      num_tokens < 0)
    return TKS_ERR_VALUE;
  if (layer_index < 0 || layer_index >= num_layers) return TKS_ERR_INDEX;
  if (num_tokens == 0) return TKS_OK;
  if (!key || !value || !key_cache || !value_cache || !slot_mapping) return TKS_ERR_VALUE;
  const PoolGeom g = make_geom(num_blocks, num_kv_heads, block_size, head_dim);
  const int64_t base = g.layer_stride * layer_index;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TKS_FLOAT32:
      return launch_append<float>(key, key_token_stride, key_head_stride, value,
                                  value_token_stride, value_head_stride, num_tokens, key_cache,
                                  value_cache, g, base, slot_mapping, s);
    case TKS_FLOAT16:
      return launch_append<_Float16>(key, key_token_stride, key_head_stride, value,
                                     value_token_stride, value_head_stride, num_tokens,
                                     key_cache, value_cache, g, base, slot_mapping, s);
    default:
      return launch_append<bf16_t>(key, key_token_stride, key_head_stride, value,
                                   value_token_stride, value_head_stride, num_tokens, key_cache,
                                   value_cache, g, base, slot_mapping, s);
  }
}

extern "C" int32_t tks_paged_gather(const void *key_cache, const void *value_cache,
                                    int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
                                    int32_t block_size, int32_t head_dim, int32_t layer_index,
                                    const int32_t *block_tables, int32_t block_table_stride,
                                    const int32_t *seq_lens, const int32_t *cu_seqlens,
                                    int32_t num_seqs, int32_t max_seq_len, void *key_out,
                                    void *value_out, int64_t out_token_stride,
                                    int64_t out_head_stride, int32_t dtype,
                                    tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (!pool_args_ok(num_layers, num_blocks, num_kv_heads, block_size, head_dim) ||
      num_seqs < 0 || max_seq_len < 0 || block_table_stride < 0)
    return TKS_ERR_VALUE;
  if (layer_index < 0 || layer_index >= num_layers) return TKS_ERR_INDEX;
  if (num_seqs == 0 || max_seq_len == 0) return TKS_OK;
  if (ceil_div(max_seq_len, block_size) > block_table_stride) return TKS_ERR_VALUE;
  if (!key_cache || !value_cache || !block_tables || !seq_lens || !cu_seqlens || !key_out ||
      !value_out)
    return TKS_ERR_VALUE;
  const PoolGeom g = make_geom(num_blocks, num_kv_heads, block_size, head_dim);
  const int64_t base = g.layer_stride * layer_index;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TKS_FLOAT32:
      return launch_gather<float>(key_cache, value_cache, g, base, num_blocks, block_tables,
                                  block_table_stride, seq_lens, cu_seqlens, num_seqs,
                                  max_seq_len, key_out, value_out, out_token_stride,
                                  out_head_stride, s);
    case TKS_FLOAT16:
      return launch_gather<_Float16>(key_cache, value_cache, g, base, num_blocks, block_tables,
                                     block_table_stride, seq_lens, cu_seqlens, num_seqs,
                                     max_seq_len, key_out, value_out, out_token_stride,
                                     out_head_stride, s);
    default:
      return launch_gather<bf16_t>(key_cache, value_cache, g, base, num_blocks, block_tables,
                                   block_table_stride, seq_lens, cu_seqlens, num_seqs,
                                   max_seq_len, key_out, value_out, out_token_stride,
                                   out_head_stride, s);
  }
}

extern "C" int32_t tks_kv_append_fp8(const void *key, int64_t key_token_stride,
                                     int64_t key_head_stride, const void *value,
                                     int64_t value_token_stride, int64_t value_head_stride,
                                     int64_t num_tokens, void *key_cache, void *value_cache,
                                     int32_t num_layers, int64_t num_blocks,
                                     int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
                                     int32_t layer_index, const int64_t *slot_mapping,
                                     float k_scale, float v_scale, int32_t dtype,
                                     tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (!pool_args_ok(num_layers, num_blocks, num_kv_heads, block_size, head_dim) ||
      num_tokens < 0 || !valid_scale(k_scale) || !valid_scale(v_scale))
    return TKS_ERR_VALUE;
  if (layer_index < 0 || layer_index >= num_layers) return TKS_ERR_INDEX;
  if (num_tokens == 0) return TKS_OK;
  if (!key || !value || !key_cache || !value_cache || !slot_mapping) return TKS_ERR_VALUE;
  const PoolGeom g = make_geom(num_blocks, num_kv_heads, block_size, head_dim);
  const int64_t base = g.layer_stride * layer_index;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define TKS_APPEND8(TYPE)                                                                     \
  launch_append_fp8<TYPE>(key, key_token_stride, key_head_stride, value, value_token_stride, \
                          value_head_stride, num_tokens, key_cache, value_cache, g, base,    \
                          slot_mapping, k_scale, v_scale, s)
  switch (dtype) {
    case TKS_FLOAT32: return TKS_APPEND8(float);
    case TKS_FLOAT16: return TKS_APPEND8(_Float16);
    default: return TKS_APPEND8(bf16_t);
  }
#undef TKS_APPEND8
}

extern "C" int32_t tks_paged_gather_fp8(const void *key_cache, const void *value_cache,
                                        int32_t num_layers, int64_t num_blocks,
                                        int32_t num_kv_heads, int32_t block_size,
                                        int32_t head_dim, int32_t layer_index,
                                        const int32_t *block_tables, int32_t block_table_stride,
                                        const int32_t *seq_lens, const int32_t *cu_seqlens,
                                        int32_t num_seqs, int32_t max_seq_len, void *key_out,
                                        void *value_out, int64_t out_token_stride,
                                        int64_t out_head_stride, float k_scale, float v_scale,
                                        int32_t dtype, tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (!pool_args_ok(num_layers, num_blocks, num_kv_heads, block_size, head_dim) ||
      num_seqs < 0 || max_seq_len < 0 || block_table_stride < 0 || !valid_scale(k_scale) ||
      !valid_scale(v_scale))
    return TKS_ERR_VALUE;
  if (layer_index < 0 || layer_index >= num_layers) return TKS_ERR_INDEX;
  if (num_seqs == 0 || max_seq_len == 0) return TKS_OK;
  if (ceil_div(max_seq_len, block_size) > block_table_stride) return TKS_ERR_VALUE;
  if (!key_cache || !value_cache || !block_tables || !seq_lens || !cu_seqlens || !key_out ||
      !value_out)
    return TKS_ERR_VALUE;
  const PoolGeom g = make_geom(num_blocks, num_kv_heads, block_size, head_dim);
  const int64_t base = g.layer_stride * layer_index;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define TKS_GATHER8(TYPE)                                                                     \
  launch_gather_fp8<TYPE>(key_cache, value_cache, g, base, num_blocks, block_tables,         \
                          block_table_stride, seq_lens, cu_seqlens, num_seqs, max_seq_len,   \
                          key_out, value_out, out_token_stride, out_head_stride, k_scale,    \
                          v_scale, s)
  switch (dtype) {
    case TKS_FLOAT32: return TKS_GATHER8(float);
    case TKS_FLOAT16: return TKS_GATHER8(_Float16);
    default: return TKS_GATHER8(bf16_t);
  }
#undef TKS_GATHER8
}
