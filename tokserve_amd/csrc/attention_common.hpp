// Pieces shared by the paged-attention kernels: pool addressing, MFMA operand
// types, split-K arrival/merge, and the argument blocks of the launchers.
//
// Scores are kept in the log2 domain: s2 = (q.k) * scale * log2(e), p = 2^(s2 - m).
#pragma once

#include "common.hpp"

namespace tks {

constexpr float kLog2e = 1.4426950408889634f;

struct PoolView {
  int64_t layer_base;    // layer * NB * Hkv * BS * Dh
  int64_t block_stride;  // Hkv * BS * Dh
  int64_t head_stride;   // BS * Dh
  int64_t num_blocks;
  int32_t block_size;
  int32_t head_dim;
};

// Block id clamped into the pool, so a corrupt table entry cannot address
// memory outside it.
__device__ __forceinline__ int64_t clamp_block(int64_t blk, int64_t num_blocks) {
  blk = blk < 0 ? 0 : blk;
  return blk >= num_blocks ? num_blocks - 1 : blk;
}

__device__ __forceinline__ int64_t block_of(const int32_t *__restrict__ bt_row, int64_t page,
                                            int64_t num_blocks) {
  return clamp_block(bt_row[page], num_blocks);
}

// NaN-propagating maximum (IEEE maximum, v_maximum3_f32 on gfx950). Unlike
// fmaxf it needs no quieting of its inputs, so a tree of them is one
// instruction per two or three values.
__device__ __forceinline__ float nan_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// 2^x on the hardware exp unit (flushes results below 2^-126 to zero, exact at -inf).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Merged output element of one (row, head, dim) from n_splits partials at w.
// Up to kMergeBatch splits are read in one batch (every load issued before the
// first is used), so such a merge costs one memory latency; longer ones read
// kMergeBatch splits at a time, the maxima first and then the sums. The
// arithmetic runs in split order either way.
constexpr int kMergeBatch = 16;
__device__ __forceinline__ float merge_splits(const float *__restrict__ ws_m,
                                              const float *__restrict__ ws_l,
                                              const float *__restrict__ ws_acc, int64_t w,
                                              int n_splits, int head_dim, int d, float *inv_l) {
  if (n_splits <= kMergeBatch) {
    float mv[kMergeBatch], lv[kMergeBatch], av[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const bool in = u < n_splits;
      mv[u] = in ? ws_m[w + u] : -INFINITY;
      lv[u] = in ? ws_l[w + u] : 0.f;
      av[u] = in ? ws_acc[(w + u) * head_dim + d] : 0.f;
    }
    float M = -INFINITY;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) M = fmaxf(M, mv[u]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      if (u < n_splits) {
        const float e = exp2f(mv[u] - M);
        L += e * lv[u];
        o += e * av[u];
      }
    }
    *inv_l = 1.f / L;
    return o;
  }
  float M = -INFINITY;
  for (int s0 = 0; s0 < n_splits; s0 += kMergeBatch) {
    float mv[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) mv[u] = s0 + u < n_splits ? ws_m[w + s0 + u] : -INFINITY;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) M = fmaxf(M, mv[u]);
  }
  float L = 0.f, o = 0.f;
  for (int s0 = 0; s0 < n_splits; s0 += kMergeBatch) {
    float mv[kMergeBatch], lv[kMergeBatch], av[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const bool in = s0 + u < n_splits;
      mv[u] = in ? ws_m[w + s0 + u] : 0.f;
      lv[u] = in ? ws_l[w + s0 + u] : 0.f;
      av[u] = in ? ws_acc[(w + s0 + u) * head_dim + d] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      if (s0 + u < n_splits) {
        const float e = exp2f(mv[u] - M);
        L += e * lv[u];
        o += e * av[u];
      }
    }
  }
  *inv_l = 1.f / L;
  return o;
}

typedef __attribute__((address_space(3))) void lds_void;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Byte address of an LDS object, as LDS instructions take it.
template <typename P>
__device__ __forceinline__ uint32_t lds_address(P *p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void *)(p)));
}

// One 16-byte HBM -> LDS load per lane: lane i's bytes land at lds + 16 * i
// (lds is wave-uniform). The compiler cannot tell which LDS bytes such a load
// writes, so it makes every later LDS access of the wave wait for all of them;
// kernels that keep such loads in flight read their LDS through inline asm.
// AUX is the load's cache policy (kLdsNonTemporal: data read once, streamed).
constexpr int kLdsNonTemporal = 2;
template <int AUX = 0>
__device__ __forceinline__ void load_lds16(const void *src, void *lds) {
#if __HIP_DEVICE_COMPILE__
  __builtin_amdgcn_global_load_lds(src, (lds_void *)lds, 16, 0, AUX);
#endif
}

// The same with 4 bytes per lane: lane i's bytes land at lds + 4 * i.
template <int AUX = 0>
__device__ __forceinline__ void load_lds4(const void *src, void *lds) {
#if __HIP_DEVICE_COMPILE__
  __builtin_amdgcn_global_load_lds(src, (lds_void *)lds, 4, 0, AUX);
#endif
}

// Max and sum over lanes l, l^16, l^32, l^48 (the four k-groups of an MFMA
// operand row), with the gfx950 cross-row lane swaps.
//
// The gfx950-only builtins and asm sit behind __HIP_DEVICE_COMPILE__: the
// host pass instantiates the kernel templates too, and a target builtin it
// does not know silently drops the kernel's launch stub.
__device__ __forceinline__ float xgroup_max(float x) {
#if __HIP_DEVICE_COMPILE__
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = nan_max(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = nan_max(__uint_as_float(b[0]), __uint_as_float(b[1]));
#endif
  return x;
}
__device__ __forceinline__ float xgroup_sum(float x) {
#if __HIP_DEVICE_COMPILE__
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(b[0]) + __uint_as_float(b[1]);
#endif
  return x;
}

template <typename T>
struct Mfma;
template <>
struct Mfma<bf16_t> {
  typedef __bf16 elem;
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef float f4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f4 run(v8 a, v8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  typedef __bf16 v4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f4 run16(v4 a, v4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<_Float16> {
  typedef _Float16 elem;
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef float f4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f4 run(v8 a, v8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  typedef _Float16 v4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f4 run16(v4 a, v4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
};

template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 as_v8(uint4 v) {
  typename Mfma<T>::v8 r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// Decode grids put the split index in the slowest dimension: every split-0
// workgroup (one per (sequence, KV head), all of them real) is dispatched
// before any later split, most of which are empty for short sequences (their
// workgroups find no keys and exit). Mixing the empty ones in between would
// leave regular gaps in the round-robin placement over XCDs and CUs.
constexpr int32_t kMaxGridSplits = 65535;

struct DecodeArgs {
  const void *q;
  int64_t q_ss, q_hs;
  const void *kc, *vc;
  PoolView pool;
  const int32_t *bt;
  int32_t bt_stride;
  const int32_t *seq_lens;
  const int32_t *seq_order;  // workgroup z -> sequence (null: identity)
  int32_t num_q_heads;
  float scale_log2;
  int32_t pages_per_split;
  int32_t max_splits;
  int32_t key_cap;  // keys any sequence may have: min(table width, splits * split size) * BS
  void *out;
  int64_t o_ss, o_hs;
  float *ws_m, *ws_l, *ws_acc;
  float v_scale = 1.f;  // V decode factor of fp8 pools (1 otherwise)
  // fp8 pools with one scale per pool row ([L, NB, Hkv, BS]; null: per-pool scales).
  const float *k_rs = nullptr, *v_rs = nullptr;
  // RoPE + KV append fused into the decode (launch_decode_mfma with rope = true):
  // sequence b's query is rotated in registers at positions[b] (q itself is not
  // written); its new key row (rotated) and value row go to pool slot slots[b]
  // (negative: none), written by the wave that reads the sequence's last page (over
  // e4m3 pools quantized with k_scale and v_scale).
  const int64_t *positions = nullptr;
  const void *cos_t = nullptr, *sin_t = nullptr;  // [table_len, Dh / 2] in the model dtype
  int64_t table_len = 0;
  const void *k_new = nullptr, *v_new = nullptr;
  int64_t kn_ss = 0, kn_hs = 0, vn_ss = 0, vn_hs = 0;
  const int64_t *slots = nullptr;
  float k_scale = 1.f;  // e4m3 pools: the new key row is stored as e4m3(key / k_scale)
};

// fp8 pools with one fp32 scale per pool row (token, KV head): the row's scale is
// amax / 448, amax its largest |x| (NaN once any value is NaN), and 1 where that
// quotient is 0, NaN or infinite.
constexpr float kE4m3Largest = 448.f;

// Largest |x| so far, NaN once any value is NaN.
__device__ __forceinline__ float abs_max_nan(float m, float x) {
  const float ax = fabsf(x);
  return (m != m || ax != ax) ? __builtin_nanf("") : fmaxf(m, ax);
}

// The same over the 64 lanes of a wave (every lane active).
__device__ __forceinline__ float wave_abs_max(float m) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = abs_max_nan(m, __shfl_xor(m, o, 64));
  return m;
}

__device__ __forceinline__ float row_scale_of(float amax) {
  const float s = amax / kE4m3Largest;
  return (s > 0.f && s < INFINITY) ? s : 1.f;
}

struct PrefillArgs {
  const void *q;
  int64_t q_ts, q_hs;  // token and head strides of the packed query
  const void *kc, *vc;
  PoolView pool;
  const int32_t *bt;
  int32_t bt_stride;
  const int32_t *seq_lens;
  const int32_t *cu_q;
  float scale_log2;
  int32_t key_cap;
  void *out;
  int64_t o_ts, o_hs;
  int32_t num_kv_heads;
  int32_t num_pairs;  // sequences * KV heads
  int32_t tiles;      // query tiles per (sequence, KV head): ceil(max_query_len / tile)
  float v_scale = 1.f;  // V decode factor (pages decoded from fp8 pools; 1 otherwise)
  const int32_t *seq_order = nullptr;  // rank -> sequence (null: identity)
  int32_t num_seqs = 0;
};

// 16-key pages of one sequence the MFMA prefill kernel holds in LDS: it serves
// sequences of up to kPrefillBtWindow * 16 keys.
constexpr int kPrefillBtWindow = 4096;

// Shapes the MFMA prefill kernel is instantiated for: block sizes that are
// multiples of 16, key_cap keys per sequence at most.
bool prefill_mfma_supported(int32_t dtype, int32_t head_dim, int32_t group, int32_t key_cap,
                            int32_t block_size, int64_t num_blocks, int32_t num_kv_heads);

// Launches the MFMA prefill kernel over grid (query tiles, Hkv, B); returns a tks_status.
int32_t launch_prefill_mfma(const PrefillArgs &a, int32_t dtype, int32_t num_seqs,
                            int32_t num_kv_heads, int32_t group, int32_t head_dim,
                            int32_t max_query_len, hipStream_t stream);

// Shapes the MFMA decode kernel is instantiated for (block size 16).
bool decode_mfma_supported(int32_t dtype, int32_t head_dim, int32_t group);

// Launches the MFMA decode kernel over grid (max_splits, Hkv, B); returns a tks_status.
// With max_splits == 1 it writes the output, otherwise split partials to be merged.
// fp8_pools: K/V pools hold e4m3 (DecodeArgs.scale_log2 then carries k_scale,
// DecodeArgs.v_scale the V factor).
int32_t launch_decode_mfma(const DecodeArgs &a, int32_t dtype, int32_t num_seqs,
                           int32_t num_kv_heads, int32_t group, int32_t head_dim,
                           hipStream_t stream, bool fp8_pools);

}  // namespace tks
