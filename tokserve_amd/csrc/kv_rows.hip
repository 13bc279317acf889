// fp8 K/V pools with one fp32 scale per pool row: the quantizing appends (plain,
// and with the step's RoPE fused in) and the decoding block-table gather.
//
// A row is one token's Dh values of one KV head. Its scale is s = amax / 448
// (amax the largest |x_d|, NaN if any x_d is NaN; s = 1 where that is 0, NaN or
// infinite), its codes e4m3(clamp(x / s, -448, 448)) with the pool encoder of
// common.hpp, and the scale goes to the row's slot of the [L, NB, Hkv, BS]
// scale array. One wave quantizes one row: each lane takes the row's elements
// d = lane + 64 j (with the RoPE fused in, the rotation pairs (d, d + Dh/2)),
// the row maximum is a wave reduction, and the codes are stored as bytes.
#include "attention_common.hpp"
#include "rope_common.hpp"

namespace tks {
namespace {

constexpr int kRowThreads = 256;
constexpr int kRowWaves = kRowThreads / 64;
constexpr int kMaxRowDh = 256;  // elements per lane: Dh / 64 <= 4

struct RowsArgs {
  // New rows (in the model dtype): key and value per token and KV head.
  const void *k;
  int64_t k_ts, k_hs;
  const void *v;
  int64_t v_ts, v_hs;
  // Pools (codes) and their scale arrays; offsets in elements of the layer.
  uint8_t *kc, *vc;
  float *ks, *vs;
  int64_t layer_base, block_stride, head_stride, num_slots;
  int32_t block_size, num_kv_heads, head_dim;
  const int64_t *slots;
  // With the RoPE fused in: the query rows rotated into qo, the key rows rotated
  // before they are quantized (and written to ko when it is given).
  const void *q;
  void *qo;
  int64_t q_ts, q_hs, qo_ts, qo_hs;
  int32_t num_q_heads;
  void *ko;
  int64_t ko_ts, ko_hs;
  const int64_t *positions;
  const void *cos_t, *sin_t;
  int64_t table_len;
};

// One workgroup per token: its query heads are rotated (RoPE), then waves take
// its 2 Hkv K and V rows, one row at a time.
template <typename T, bool ROPE>
__global__ __launch_bounds__(kRowThreads) void append_rows_kernel(RowsArgs a) {
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int DH = a.head_dim;
  const int HALF = DH / 2;
  const T *crow = nullptr;
  const T *srow = nullptr;
  if constexpr (ROPE) {
    int64_t pos = a.positions[t];
    pos = pos < 0 ? 0 : (pos >= a.table_len ? a.table_len - 1 : pos);
    crow = static_cast<const T *>(a.cos_t) + pos * HALF;
    srow = static_cast<const T *>(a.sin_t) + pos * HALF;
    for (int i = threadIdx.x; i < a.num_q_heads * HALF; i += kRowThreads) {
      const int h = i / HALF, d = i - (i / HALF) * HALF;
      const T *src = static_cast<const T *>(a.q) + t * a.q_ts + h * a.q_hs;
      T *dst = static_cast<T *>(a.qo) + t * a.qo_ts + h * a.qo_hs;
      const float x1 = to_float(src[d]), x2 = to_float(src[d + HALF]);
      const float c = to_float(crow[d]), s = to_float(srow[d]);
      float o1, o2;
      rotate_math<T, 1>(&x1, &x2, &c, &s, &o1, &o2);
      dst[d] = from_float<T>(o1);
      dst[d + HALF] = from_float<T>(o2);
    }
  }
  const int64_t slot = a.slots[t];
  const bool keep = slot >= 0 && slot < a.num_slots;
  int64_t row_base = 0;  // element offset of the slot's row of KV head 0
  if (keep) {
    const int64_t block = slot / a.block_size;
    row_base = a.layer_base + block * a.block_stride + (slot - block * a.block_size) * DH;
  }
  const int H = a.num_kv_heads;
  for (int r = wave; r < 2 * H; r += kRowWaves) {
    const bool is_k = r < H;
    const int h = is_k ? r : r - H;
    // This lane's elements of the row: index e[j] = lane + 64 j, or with the
    // rotation the pairs (lane + 64 j, lane + 64 j + HALF).
    constexpr int J = kMaxRowDh / 64;
    float x[J];
    int e[J];
    bool ok[J];
    if (ROPE && is_k) {
      const T *src = static_cast<const T *>(a.k) + t * a.k_ts + h * a.k_hs;
      T *kout = a.ko ? static_cast<T *>(a.ko) + t * a.ko_ts + h * a.ko_hs : nullptr;
#pragma unroll
      for (int j = 0; j < J / 2; ++j) {
        const int d = lane + 64 * j;
        ok[2 * j] = ok[2 * j + 1] = d < HALF;
        x[2 * j] = x[2 * j + 1] = 0.f;
        e[2 * j] = d;
        e[2 * j + 1] = d + HALF;
        if (d < HALF) {
          const float x1 = to_float(src[d]), x2 = to_float(src[d + HALF]);
          const float c = to_float(crow[d]), s = to_float(srow[d]);
          float o1, o2;
          rotate_math<T, 1>(&x1, &x2, &c, &s, &o1, &o2);
          // The rotated row at the model dtype's precision, as the two-step path
          // stores it before the quantizing append reads it.
          o1 = round_through<T>(o1);
          o2 = round_through<T>(o2);
          if (kout) {
            kout[d] = from_float<T>(o1);
            kout[d + HALF] = from_float<T>(o2);
          }
          x[2 * j] = o1;
          x[2 * j + 1] = o2;
        }
      }
    } else {
      const T *src = is_k ? static_cast<const T *>(a.k) + t * a.k_ts + h * a.k_hs
                          : static_cast<const T *>(a.v) + t * a.v_ts + h * a.v_hs;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int d = lane + 64 * j;
        ok[j] = d < DH;
        e[j] = d;
        x[j] = d < DH ? to_float(src[d]) : 0.f;
      }
    }
    if (!keep) continue;
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (ok[j]) amax = abs_max_nan(amax, x[j]);
    const float s = row_scale_of(wave_abs_max(amax));
    uint8_t *dst = (is_k ? a.kc : a.vc) + row_base + h * a.head_stride;
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (ok[j]) dst[e[j]] = e4m3_code(x[j], s);
    if (lane == 0) (is_k ? a.ks : a.vs)[(row_base + h * a.head_stride) / DH] = s;
  }
}

// Decoding gather: one thread per element of the gathered rows.
template <typename T>
__global__ __launch_bounds__(256) void gather_rows_kernel(
    const uint8_t *__restrict__ kc, const uint8_t *__restrict__ vc, const float *__restrict__ ks,
    const float *__restrict__ vs, int64_t layer_base, int64_t block_stride, int64_t head_stride,
    int32_t block_size, int32_t num_kv_heads, int32_t head_dim, int64_t num_blocks,
    const int32_t *__restrict__ bt, int32_t bt_stride, const int32_t *__restrict__ seq_lens,
    const int32_t *__restrict__ cu, int32_t max_seq_len, T *__restrict__ k_out,
    T *__restrict__ v_out, int64_t o_ts, int64_t o_hs) {
  const int b = blockIdx.y;
  const int64_t per_token = static_cast<int64_t>(num_kv_heads) * head_dim;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t p = item / per_token;
  if (p >= max_seq_len || p >= seq_lens[b]) return;
  const int rem = static_cast<int>(item - p * per_token);
  const int h = rem / head_dim;
  const int d = rem - h * head_dim;
  const int64_t block = bt[static_cast<int64_t>(b) * bt_stride + p / block_size];
  if (block < 0 || block >= num_blocks) return;
  const int64_t row = layer_base + block * block_stride + h * head_stride + (p % block_size) * head_dim;
  const int64_t dst = (cu[b] + p) * o_ts + h * o_hs + d;
  // The fp32 product, then one rounding to T.
  k_out[dst] = from_float<T>(fp32_value(to_float(fp8e4m3_t{kc[row + d]}) * ks[row / head_dim]));
  v_out[dst] = from_float<T>(fp32_value(to_float(fp8e4m3_t{vc[row + d]}) * vs[row / head_dim]));
}

bool pool_args_ok(int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
                  int32_t block_size, int32_t head_dim, int32_t layer_index) {
  return num_layers > 0 && num_blocks > 0 && num_kv_heads > 0 && block_size > 0 &&
         head_dim > 0 && head_dim <= kMaxRowDh && layer_index >= 0;
}

int32_t launch_rows(RowsArgs a, bool rope, int64_t num_tokens, int32_t dtype, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(num_tokens));
#define TKS_ROWS(TYPE)                                                  \
  if (rope)                                                             \
    append_rows_kernel<TYPE, true><<<grid, kRowThreads, 0, s>>>(a);     \
  else                                                                  \
    append_rows_kernel<TYPE, false><<<grid, kRowThreads, 0, s>>>(a)
  switch (dtype) {
    case TKS_FLOAT32: TKS_ROWS(float); break;
    case TKS_FLOAT16: TKS_ROWS(_Float16); break;
    default: TKS_ROWS(bf16_t); break;
  }
#undef TKS_ROWS
  return check_launch();
}

RowsArgs pool_rows(void *key_cache, void *value_cache, float *k_scales, float *v_scales,
                   int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
                   int32_t head_dim, int32_t layer_index, const int64_t *slots) {
  RowsArgs a{};
  a.kc = static_cast<uint8_t *>(key_cache);
  a.vc = static_cast<uint8_t *>(value_cache);
  a.ks = k_scales;
  a.vs = v_scales;
  a.head_stride = static_cast<int64_t>(block_size) * head_dim;
  a.block_stride = a.head_stride * num_kv_heads;
  a.layer_base = a.block_stride * num_blocks * layer_index;
  a.num_slots = num_blocks * block_size;
  a.block_size = block_size;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.slots = slots;
  return a;
}

}  // namespace
}  // namespace tks

using namespace tks;

extern "C" int32_t tks_kv_append_fp8_rows(const void *key, int64_t key_token_stride,
                                          int64_t key_head_stride, const void *value,
                                          int64_t value_token_stride, int64_t value_head_stride,
                                          int64_t num_tokens, void *key_cache, void *value_cache,
                                          float *k_scales, float *v_scales, int32_t num_layers,
                                          int64_t num_blocks, int32_t num_kv_heads,
                                          int32_t block_size, int32_t head_dim,
                                          int32_t layer_index, const int64_t *slot_mapping,
                                          int32_t dtype, tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (!pool_args_ok(num_layers, num_blocks, num_kv_heads, block_size, head_dim, 0) ||
      num_tokens < 0)
    return TKS_ERR_VALUE;
  if (layer_index < 0 || layer_index >= num_layers) return TKS_ERR_INDEX;
  if (num_tokens == 0) return TKS_OK;
  if (num_tokens > 0x7fffffff) return TKS_ERR_VALUE;
  if (!key || !value || !key_cache || !value_cache || !k_scales || !v_scales || !slot_mapping)
    return TKS_ERR_VALUE;
  RowsArgs a = pool_rows(key_cache, value_cache, k_scales, v_scales, num_blocks, num_kv_heads,
                         block_size, head_dim, layer_index, slot_mapping);
  a.k = key;
  a.k_ts = key_token_stride;
  a.k_hs = key_head_stride;
  a.v = value;
  a.v_ts = value_token_stride;
  a.v_hs = value_head_stride;
  return launch_rows(a, false, num_tokens, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int32_t tks_rope_kv_append_fp8_rows(
    const void *query, void *query_out, int64_t q_ts, int64_t q_hs, int64_t qo_ts,
    int64_t qo_hs, int32_t num_q_heads, const void *key, void *key_out, int64_t k_ts,
    int64_t k_hs, int64_t ko_ts, int64_t ko_hs, const void *value, int64_t v_ts, int64_t v_hs,
    int32_t num_kv_heads, int64_t num_tokens, int32_t head_dim, const int64_t *positions,
    const void *cos_cache, const void *sin_cache, int64_t cache_len, void *key_cache,
    void *value_cache, float *k_scales, float *v_scales, int32_t num_layers, int64_t num_blocks,
    int32_t block_size, int32_t layer_index, const int64_t *slot_mapping, int32_t dtype,
    tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (!pool_args_ok(num_layers, num_blocks, num_kv_heads, block_size, head_dim, 0) ||
      head_dim < 2 || head_dim % 2 != 0 || num_q_heads < 0 || num_tokens < 0 || cache_len <= 0)
    return TKS_ERR_VALUE;
  if (layer_index < 0 || layer_index >= num_layers) return TKS_ERR_INDEX;
  if (num_tokens == 0) return TKS_OK;
  if (num_tokens > 0x7fffffff) return TKS_ERR_VALUE;
  if ((num_q_heads > 0 && (!query || !query_out)) || !key || !value || !positions ||
      !cos_cache || !sin_cache || !key_cache || !value_cache || !k_scales || !v_scales ||
      !slot_mapping)
    return TKS_ERR_VALUE;
  RowsArgs a = pool_rows(key_cache, value_cache, k_scales, v_scales, num_blocks, num_kv_heads,
                         block_size, head_dim, layer_index, slot_mapping);
  a.k = key;
  a.k_ts = k_ts;
  a.k_hs = k_hs;
  a.v = value;
  a.v_ts = v_ts;
  a.v_hs = v_hs;
  a.q = query;
  a.qo = query_out;
  a.q_ts = q_ts;
  a.q_hs = q_hs;
  a.qo_ts = qo_ts;
  a.qo_hs = qo_hs;
  a.num_q_heads = num_q_heads;
  a.ko = key_out;
  a.ko_ts = ko_ts;
  a.ko_hs = ko_hs;
  a.positions = positions;
  a.cos_t = cos_cache;
  a.sin_t = sin_cache;
  a.table_len = cache_len;
  return launch_rows(a, true, num_tokens, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int32_t tks_paged_gather_fp8_rows(
    const void *key_cache, const void *value_cache, const float *k_scales, const float *v_scales,
    int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
    int32_t head_dim, int32_t layer_index, const int32_t *block_tables, int32_t block_table_stride,
    const int32_t *seq_lens, const int32_t *cu_seqlens, int32_t num_seqs, int32_t max_seq_len,
    void *key_out, void *value_out, int64_t out_token_stride, int64_t out_head_stride,
    int32_t dtype, tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (!pool_args_ok(num_layers, num_blocks, num_kv_heads, block_size, head_dim, 0) ||
      num_seqs < 0 || max_seq_len < 0 || block_table_stride < 0)
    return TKS_ERR_VALUE;
  if (layer_index < 0 || layer_index >= num_layers) return TKS_ERR_INDEX;
  if (num_seqs == 0 || max_seq_len == 0) return TKS_OK;
  if (num_seqs > 65535 || ceil_div(max_seq_len, block_size) > block_table_stride) return TKS_ERR_VALUE;
  if (!key_cache || !value_cache || !k_scales || !v_scales || !block_tables || !seq_lens ||
      !cu_seqlens || !key_out || !value_out)
    return TKS_ERR_VALUE;
  const int64_t head_stride = static_cast<int64_t>(block_size) * head_dim;
  const int64_t block_stride = head_stride * num_kv_heads;
  const int64_t layer_base = block_stride * num_blocks * layer_index;
  const int64_t items = static_cast<int64_t>(max_seq_len) * num_kv_heads * head_dim;
  if (ceil_div(items, 256) > 0x7fffffff) return TKS_ERR_VALUE;
  const dim3 grid(static_cast<unsigned>(ceil_div(items, 256)), num_seqs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t *kc = static_cast<const uint8_t *>(key_cache);
  const uint8_t *vc = static_cast<const uint8_t *>(value_cache);
#define TKS_GATHER_ROWS(TYPE)                                                                 \
  gather_rows_kernel<TYPE><<<grid, 256, 0, s>>>(                                              \
      kc, vc, k_scales, v_scales, layer_base, block_stride, head_stride, block_size,           \
      num_kv_heads, head_dim, num_blocks, block_tables, block_table_stride, seq_lens,          \
      cu_seqlens, max_seq_len, static_cast<TYPE *>(key_out), static_cast<TYPE *>(value_out),   \
      out_token_stride, out_head_stride)
  switch (dtype) {
    case TKS_FLOAT32: TKS_GATHER_ROWS(float); break;
    case TKS_FLOAT16: TKS_GATHER_ROWS(_Float16); break;
    default: TKS_GATHER_ROWS(bf16_t); break;
  }
#undef TKS_GATHER_ROWS
  return check_launch();
}
