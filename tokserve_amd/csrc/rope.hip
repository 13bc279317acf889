// Half-rotation RoPE on Q and K of a packed (or (B, H, T, Dh)) token stream.
//
//   out[d]        = r(x[d]        * cos[d]) + r(-x[d + D/2] * sin[d])
//   out[d + D/2]  = r(x[d + D/2]  * cos[d]) + r( x[d]       * sin[d])      (d < D/2)
//
// with every product rounded to the element type before the add, as
// tokserve/kernels/_triton_rope.py:63-66 and apply_rope (tokserve/engine/rope.py:150-153)
// do. cos/sin rows come from a per-position table already cast to the element
// type (tokserve/engine/rope.py:78-87), so the kernel only gathers and rotates.
// One workgroup per token: the table row is read once and shared by all
// Hq + Hkv heads; each lane rotates one 16-byte chunk of the first half
// together with its partner chunk of the second half.
#include "rope_common.hpp"

namespace tks {
namespace {

constexpr int kThreads = 128;
// The fused RoPE + KV append has more work per token (the V rows too): a decode
// token of the TinyLlama shape is 176 16-byte items, one round for 256 threads
// (128 x 176 items: 3.74 -> 3.12 us graph-timed).
constexpr int kAppendThreads = 256;

struct RopeTensor {
  const void *in;
  void *out;
  int64_t sb, sh, st;     // input strides (batch, head, token)
  int64_t osb, osh, ost;  // output strides
  int32_t heads;
};

template <typename T, int V>
__device__ __forceinline__ void rotate(const T *x, T *y, const float *c, const float *s,
                                       int half) {
  float o1[V], o2[V];
  rotate_values<T, V>(x, c, s, half, o1, o2);
  store_pair<T, V>(y, o1, o2, half);
}

template <typename T, int V>
__global__ __launch_bounds__(kThreads) void rope_kernel(RopeTensor q, RopeTensor k,
                                                        const int64_t *__restrict__ positions,
                                                        const T *__restrict__ cos_cache,
                                                        const T *__restrict__ sin_cache,
                                                        int64_t cache_len, int32_t head_dim) {
  const int64_t t = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int half = head_dim / 2;
  const int chunks = half / V;
  int64_t pos = positions[t];
  pos = pos < 0 ? 0 : (pos >= cache_len ? cache_len - 1 : pos);
  const T *crow = cos_cache + pos * half;
  const T *srow = sin_cache + pos * half;
  const int items = (q.heads + k.heads) * chunks;
  if (kThreads % chunks == 0) {
    // Every item a thread visits has the same chunk: its table values are read once.
    const int c = (threadIdx.x % chunks) * V;
    float cf[V], sf[V];
    load_table<T, V>(crow, srow, c, cf, sf);
    for (int it = threadIdx.x; it < items; it += kThreads) {
      const int h = it / chunks;
      const RopeTensor &x = h < q.heads ? q : k;
      const int hh = h < q.heads ? h : h - q.heads;
      const T *src = static_cast<const T *>(x.in) + b * x.sb + hh * x.sh + t * x.st + c;
      T *dst = static_cast<T *>(x.out) + b * x.osb + hh * x.osh + t * x.ost + c;
      rotate<T, V>(src, dst, cf, sf, half);
    }
    return;
  }
  for (int it = threadIdx.x; it < items; it += kThreads) {
    const int h = it / chunks;
    const int c = (it - h * chunks) * V;
    float cf[V], sf[V];
    load_table<T, V>(crow, srow, c, cf, sf);
    const RopeTensor &x = h < q.heads ? q : k;
    const int hh = h < q.heads ? h : h - q.heads;
    const T *src = static_cast<const T *>(x.in) + b * x.sb + hh * x.sh + t * x.st + c;
    T *dst = static_cast<T *>(x.out) + b * x.osb + hh * x.osh + t * x.ost + c;
    rotate<T, V>(src, dst, cf, sf, half);
  }
}

// RoPE on a packed step's Q and K fused with the KV append: token t's rotated
// K rows go straight to pool slot slot_mapping[t] (and to k_out when given), its
// V rows are copied there, Q is rotated into q_out. One workgroup per token.
// Equal, bit for bit, to tks_rope followed by tks_kv_append on the rotated K.
struct AppendView {
  const void *v;
  int64_t v_ts, v_hs;
  void *kc, *vc;
  int64_t layer_base, block_stride, head_stride, num_slots;
  int32_t block_size;
  const int64_t *slots;
  float k_scale, v_scale;  // e4m3 pools: the codes hold value / scale
};

template <typename T, int V, typename P>
__global__ __launch_bounds__(kAppendThreads) void rope_append_kernel(
    RopeTensor q, RopeTensor k, AppendView a, const int64_t *__restrict__ positions,
    const T *__restrict__ cos_cache, const T *__restrict__ sin_cache, int64_t cache_len,
    int32_t head_dim) {
  const int64_t t = blockIdx.x;
  const int half = head_dim / 2;
  const int chunks = half / V;
  int64_t pos = positions[t];
  pos = pos < 0 ? 0 : (pos >= cache_len ? cache_len - 1 : pos);
  const T *crow = cos_cache + pos * half;
  const T *srow = sin_cache + pos * half;
  const int64_t slot = a.slots[t];
  const bool keep = slot >= 0 && slot < a.num_slots;
  int64_t row = 0;
  if (keep) {
    const int64_t block = slot / a.block_size;
    row = a.layer_base + block * a.block_stride + (slot - block * a.block_size) * head_dim;
  }
  P *kc = static_cast<P *>(a.kc);
  P *vc = static_cast<P *>(a.vc);
  const int rot_items = (q.heads + k.heads) * chunks;
  const int v_chunks = head_dim / V;
  const int items = rot_items + (keep ? k.heads * v_chunks : 0);
  for (int it = threadIdx.x; it < items; it += kAppendThreads) {
    if (it >= rot_items) {  // V copy
      const int j = it - rot_items;
      const int h = j / v_chunks;
      const int c = (j - h * v_chunks) * V;
      const T *src = static_cast<const T *>(a.v) + t * a.v_ts + h * a.v_hs + c;
      P *dst = vc + row + h * a.head_stride + c;
      if constexpr (sizeof(P) != 1 && V * sizeof(T) == 16) {
        st16(dst, ld16(src));
      } else if constexpr (sizeof(P) != 1) {
#pragma unroll
        for (int e = 0; e < V; ++e) dst[e] = src[e];
      } else {
        float x[V];
        if constexpr (V * sizeof(T) == 16) {
          unpack<T>(ld16(src), x);
        } else {
#pragma unroll
          for (int e = 0; e < V; ++e) x[e] = to_float(src[e]);
        }
        encode_e4m3<V>(x, a.v_scale, reinterpret_cast<uint8_t *>(dst));
      }
      continue;
    }
    const int h = it / chunks;
    const int c = (it - h * chunks) * V;
    float cf[V], sf[V], o1[V], o2[V];
    load_table<T, V>(crow, srow, c, cf, sf);
    if (h < q.heads) {
      const T *src = static_cast<const T *>(q.in) + h * q.sh + t * q.st + c;
      T *dst = static_cast<T *>(q.out) + h * q.osh + t * q.ost + c;
      rotate<T, V>(src, dst, cf, sf, half);
    } else {
      const int hh = h - q.heads;
      const T *src = static_cast<const T *>(k.in) + hh * k.sh + t * k.st + c;
      rotate_values<T, V>(src, cf, sf, half, o1, o2);
      if (k.out != nullptr)
        store_pair<T, V>(static_cast<T *>(k.out) + hh * k.osh + t * k.ost + c, o1, o2, half);
      if (keep) {
        if constexpr (sizeof(P) == 1) {
          // The rotated row at the model dtype's precision, as the two-step path
          // stores it before the quantizing append reads it.
#pragma unroll
          for (int e = 0; e < V; ++e) {
            o1[e] = round_through<T>(o1[e]);
            o2[e] = round_through<T>(o2[e]);
          }
          P *dst = kc + row + hh * a.head_stride + c;
          encode_e4m3<V>(o1, a.k_scale, reinterpret_cast<uint8_t *>(dst));
          encode_e4m3<V>(o2, a.k_scale, reinterpret_cast<uint8_t *>(dst + half));
        } else {
          store_pair<T, V>(kc + row + hh * a.head_stride + c, o1, o2, half);
        }
      }
    }
  }
}

bool strides_ok(const RopeTensor &x, int v) {
  return x.sb % v == 0 && x.sh % v == 0 && x.st % v == 0 && x.osb % v == 0 &&
         x.osh % v == 0 && x.ost % v == 0 && aligned16(x.in) && aligned16(x.out);
}

template <typename T>
int32_t launch(const RopeTensor &q, const RopeTensor &k, int32_t batch, int64_t tokens,
               int32_t head_dim, const int64_t *pos, const void *cc, const void *sc,
               int64_t cache_len, hipStream_t s) {
  constexpr int V = Vec<T>::N;
  const int half = head_dim / 2;
  const bool vec = half % V == 0 && aligned16(cc) && aligned16(sc) && strides_ok(q, V) &&
                   (k.heads == 0 || strides_ok(k, V));
  const dim3 grid(static_cast<unsigned>(tokens), batch);
  if (vec)
    rope_kernel<T, V><<<grid, kThreads, 0, s>>>(q, k, pos, static_cast<const T *>(cc),
                                                static_cast<const T *>(sc), cache_len, head_dim);
  else
    rope_kernel<T, 1><<<grid, kThreads, 0, s>>>(q, k, pos, static_cast<const T *>(cc),
                                                static_cast<const T *>(sc), cache_len, head_dim);
  return check_launch();
}

}  // namespace
}  // namespace tks

using namespace tks;

extern "C" int32_t tks_rope(const void *query, void *query_out, int64_t q_sb, int64_t q_sh,
                            int64_t q_st, int64_t qo_sb, int64_t qo_sh, int64_t qo_st,
                            int32_t num_q_heads, const void *key, void *key_out, int64_t k_sb,
                            int64_t k_sh, int64_t k_st, int64_t ko_sb, int64_t ko_sh,
                            int64_t ko_st, int32_t num_kv_heads, int32_t batch,
                            int64_t num_tokens, int32_t head_dim, const int64_t *positions,
                            const void *cos_cache, const void *sin_cache, int64_t cache_len,
                            int32_t dtype, tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (head_dim < 2 || head_dim % 2 != 0 || num_q_heads < 0 || num_kv_heads < 0 || batch < 0 ||
      num_tokens < 0 || cache_len <= 0)
    return TKS_ERR_VALUE;
  if (batch == 0 || num_tokens == 0 || num_q_heads + num_kv_heads == 0) return TKS_OK;
  if (num_tokens > 0x7fffffff || batch > 65535) return TKS_ERR_VALUE;
  if ((num_q_heads > 0 && (!query || !query_out)) || (num_kv_heads > 0 && (!key || !key_out)) ||
      !positions || !cos_cache || !sin_cache)
    return TKS_ERR_VALUE;
  const RopeTensor q{query, query_out, q_sb, q_sh, q_st, qo_sb, qo_sh, qo_st, num_q_heads};
  const RopeTensor k{key, key_out, k_sb, k_sh, k_st, ko_sb, ko_sh, ko_st, num_kv_heads};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TKS_FLOAT32:
      return launch<float>(q, k, batch, num_tokens, head_dim, positions, cos_cache, sin_cache,
                           cache_len, s);
    case TKS_FLOAT16:
      return launch<_Float16>(q, k, batch, num_tokens, head_dim, positions, cos_cache,
                              sin_cache, cache_len, s);
    default:
      return launch<bf16_t>(q, k, batch, num_tokens, head_dim, positions, cos_cache, sin_cache,
                            cache_len, s);
  }
}

namespace {

int32_t rope_kv_append_impl(
    const void *query, void *query_out, int64_t q_ts, int64_t q_hs, int64_t qo_ts,
    int64_t qo_hs, int32_t num_q_heads, const void *key, void *key_out, int64_t k_ts,
    int64_t k_hs, int64_t ko_ts, int64_t ko_hs, const void *value, int64_t v_ts, int64_t v_hs,
    int32_t num_kv_heads, int64_t num_tokens, int32_t head_dim, const int64_t *positions,
    const void *cos_cache, const void *sin_cache, int64_t cache_len, void *key_cache,
    void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t block_size,
    int32_t layer_index, const int64_t *slot_mapping, bool fp8_pools, float k_scale,
    float v_scale, int32_t dtype, tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (head_dim < 2 || head_dim % 2 != 0 || num_q_heads < 0 || num_kv_heads <= 0 ||
      num_tokens < 0 || cache_len <= 0 || num_layers <= 0 || num_blocks <= 0 || block_size <= 0 ||
      !valid_scale(k_scale) || !valid_scale(v_scale))
    return TKS_ERR_VALUE;
  if (layer_index < 0 || layer_index >= num_layers) return TKS_ERR_INDEX;
  if (num_tokens == 0) return TKS_OK;
  if (num_tokens > 0x7fffffff) return TKS_ERR_VALUE;
  if ((num_q_heads > 0 && (!query || !query_out)) || !key || !value || !positions ||
      !cos_cache || !sin_cache || !key_cache || !value_cache || !slot_mapping)
    return TKS_ERR_VALUE;
  const RopeTensor q{query, query_out, 0, q_hs, q_ts, 0, qo_hs, qo_ts, num_q_heads};
  const RopeTensor k{key, key_out, 0, k_hs, k_ts, 0, ko_hs, ko_ts, num_kv_heads};
  AppendView a;
  a.v = value;
  a.v_ts = v_ts;
  a.v_hs = v_hs;
  a.kc = key_cache;
  a.vc = value_cache;
  a.head_stride = static_cast<int64_t>(block_size) * head_dim;
  a.block_stride = a.head_stride * num_kv_heads;
  a.layer_base = a.block_stride * num_blocks * layer_index;
  a.num_slots = num_blocks * block_size;
  a.block_size = block_size;
  a.slots = slot_mapping;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(num_tokens));
#define TKS_ROPE_APPEND_POOL(TYPE, VV, POOL)                                                     \
  rope_append_kernel<TYPE, VV, POOL><<<grid, kAppendThreads, 0, s>>>(                           \
      q, k, a, positions, static_cast<const TYPE *>(cos_cache),                                 \
      static_cast<const TYPE *>(sin_cache), cache_len, head_dim)
#define TKS_ROPE_APPEND(TYPE)                                                                  \
  {                                                                                            \
    constexpr int V = Vec<TYPE>::N;                                                            \
    const RopeTensor kk{key, key_out ? key_out : const_cast<void *>(key), 0, k_hs, k_ts, 0,    \
                        ko_hs, ko_ts, num_kv_heads};                                           \
    const bool vec = (head_dim / 2) % V == 0 && aligned16(cos_cache) && aligned16(sin_cache) && \
                     (num_q_heads == 0 || strides_ok(q, V)) && strides_ok(kk, V) &&             \
                     v_ts % V == 0 && v_hs % V == 0 && aligned16(value) &&                      \
                     aligned16(key_cache) && aligned16(value_cache);                            \
    if (fp8_pools) {                                                                           \
      if (vec)                                                                                 \
        TKS_ROPE_APPEND_POOL(TYPE, V, fp8e4m3_t);                                              \
      else                                                                                     \
        TKS_ROPE_APPEND_POOL(TYPE, 1, fp8e4m3_t);                                              \
    } else if (vec) {                                                                          \
      TKS_ROPE_APPEND_POOL(TYPE, V, TYPE);                                                     \
    } else {                                                                                   \
      TKS_ROPE_APPEND_POOL(TYPE, 1, TYPE);                                                     \
    }                                                                                          \
  }
  switch (dtype) {
    case TKS_FLOAT32: TKS_ROPE_APPEND(float); break;
    case TKS_FLOAT16: TKS_ROPE_APPEND(_Float16); break;
    default: TKS_ROPE_APPEND(bf16_t); break;
  }
#undef TKS_ROPE_APPEND
#undef TKS_ROPE_APPEND_POOL
  return check_launch();
}

}  // namespace

extern "C" int32_t tks_rope_kv_append(
    const void *query, void *query_out, int64_t q_ts, int64_t q_hs, int64_t qo_ts,
    int64_t qo_hs, int32_t num_q_heads, const void *key, void *key_out, int64_t k_ts,
    int64_t k_hs, int64_t ko_ts, int64_t ko_hs, const void *value, int64_t v_ts, int64_t v_hs,
    int32_t num_kv_heads, int64_t num_tokens, int32_t head_dim, const int64_t *positions,
    const void *cos_cache, const void *sin_cache, int64_t cache_len, void *key_cache,
    void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t block_size,
    int32_t layer_index, const int64_t *slot_mapping, int32_t dtype, tks_stream_t stream) {
  return rope_kv_append_impl(query, query_out, q_ts, q_hs, qo_ts, qo_hs, num_q_heads, key,
                             key_out, k_ts, k_hs, ko_ts, ko_hs, value, v_ts, v_hs, num_kv_heads,
                             num_tokens, head_dim, positions, cos_cache, sin_cache, cache_len,
                             key_cache, value_cache, num_layers, num_blocks, block_size,
                             layer_index, slot_mapping, false, 1.f, 1.f, dtype, stream);
}

extern "C" int32_t tks_rope_kv_append_fp8(
    const void *query, void *query_out, int64_t q_ts, int64_t q_hs, int64_t qo_ts,
    int64_t qo_hs, int32_t num_q_heads, const void *key, void *key_out, int64_t k_ts,
    int64_t k_hs, int64_t ko_ts, int64_t ko_hs, const void *value, int64_t v_ts, int64_t v_hs,
    int32_t num_kv_heads, int64_t num_tokens, int32_t head_dim, const int64_t *positions,
    const void *cos_cache, const void *sin_cache, int64_t cache_len, void *key_cache,
    void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t block_size,
    int32_t layer_index, const int64_t *slot_mapping, float k_scale, float v_scale,
    int32_t dtype, tks_stream_t stream) {
  return rope_kv_append_impl(query, query_out, q_ts, q_hs, qo_ts, qo_hs, num_q_heads, key,
                             key_out, k_ts, k_hs, ko_ts, ko_hs, value, v_ts, v_hs, num_kv_heads,
                             num_tokens, head_dim, positions, cos_cache, sin_cache, cache_len,
                             key_cache, value_cache, num_layers, num_blocks, block_size,
                             layer_index, slot_mapping, true, k_scale, v_scale, dtype, stream);
}
