// Paged attention over block tables: decode (split-K) and ragged chunked prefill.
//
// Semantics follow tokserve/kernels/_triton_paged_attention.py:12-149: K/V are
// read through block_table[logical_block] (:76-82) from one layer of the
// [L, NB, Hkv, BS, Dh] pools, query head hq uses KV head hq / G (:49), the
// causal mask is key <= query position (:118-123), softmax is accumulated
// online in fp32 (:125-136) and the output is acc / sum in the query dtype (:138).
//
// Kernels
//   decode_mfma_kernel   bf16/fp16, BS == 16, Dh in {64, 128}, G = Hq/Hkv in {1..16}.
//       One wave per (sequence, KV head, split); each 16-token page of one KV
//       head (16 x Dh contiguous elements) is one MFMA tile. S^T = Q_rep . K^T
//       with v_mfma_f32_16x16x32_{bf16,f16}: the A operand replicates the G
//       query heads over the 16 rows, K rows feed the B operand straight from
//       16-byte HBM loads. The per-page probabilities (G x 16) go through LDS
//       so that P.V runs on the VALU with every lane owning 2 dims of G/HG
//       heads over all 16 tokens (8 fp32 accumulators at G=4): a V row is one
//       coalesced 256-byte wave load, nothing is reduced across lanes at the
//       end, and registers stay low enough for 4+ waves per SIMD. The G heads
//       share every KV byte, so each page is read from HBM exactly once; the
//       next page is prefetched into registers while the current one is used.
//   attn_generic_kernel  any dtype / block size / G <= 16 / Dh <= 128.
//       One wave per (query row, KV head, split), 64 keys per step. Used for
//       fp32 (where 1e-5 parity wants full fp32 products), odd shapes, and as
//       the ragged-prefill path (one row per query token, causal length).
//   Split-K partials (m, l, acc per head) go to the workspace; the last wave of
//   each (row, KV head) to finish merges them in place:
//       o = sum_s 2^(m_s-M) acc_s / sum_s 2^(m_s-M) l_s,   M = max_s m_s,
//   so a decode step is a single launch.
//
// Scores are kept in the log2 domain: s2 = (q.k) * scale * log2(e), p = 2^(s2 - m).
#include "common.hpp"

#include <algorithm>

namespace tks {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

struct PoolView {
  int64_t layer_base;    // layer * NB * Hkv * BS * Dh
  int64_t block_stride;  // Hkv * BS * Dh
  int64_t head_stride;   // BS * Dh
  int64_t num_blocks;
  int32_t block_size;
  int32_t head_dim;
};

// Block id of logical page `page` of a row, clamped into the pool so that a
// corrupt table can never address memory outside it.
__device__ __forceinline__ int64_t block_of(const int32_t *__restrict__ bt_row, int64_t page,
                                            int64_t num_blocks) {
  int64_t blk = bt_row[page];
  blk = blk < 0 ? 0 : blk;
  return blk >= num_blocks ? num_blocks - 1 : blk;
}

// Split-K arrival: every wave of a (row, KV head) stores its partials, then
// bumps the pair's counter. The wave that arrives last sees every partial
// (release/acquire at agent scope, across XCDs) and merges them; it also puts
// the counter back to zero, so the workspace stays ready for the next launch.
__device__ __forceinline__ bool arrive_last(int32_t *counter, int n_splits) {
  __threadfence();
  __syncthreads();
  int prev = 0;
  if (threadIdx.x == 0)
    prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0, 64);
  if (prev != n_splits - 1) return false;
  __threadfence();
  return true;
}

__device__ __forceinline__ void release_counter(int32_t *counter) {
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merged output element of one (row, head, dim) from n_splits partials at w.
__device__ __forceinline__ float merge_splits(const float *__restrict__ ws_m,
                                              const float *__restrict__ ws_l,
                                              const float *__restrict__ ws_acc, int64_t w,
                                              int n_splits, int head_dim, int d, float *inv_l) {
  float M = -INFINITY;
  for (int s = 0; s < n_splits; ++s) M = fmaxf(M, ws_m[w + s]);
  float L = 0.f, o = 0.f;
  for (int s = 0; s < n_splits; ++s) {
    const float e = exp2f(ws_m[w + s] - M);
    L += e * ws_l[w + s];
    o += e * ws_acc[(w + s) * head_dim + d];
  }
  *inv_l = 1.f / L;
  return o;
}

// ------------------------------------------------------------------------
// MFMA decode kernel
// ------------------------------------------------------------------------

template <typename T>
struct Mfma;
template <>
struct Mfma<bf16_t> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ float4 run(v8 a, v8 b, float4 c) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    f4 r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, f4{c.x, c.y, c.z, c.w}, 0, 0, 0);
    return make_float4(r[0], r[1], r[2], r[3]);
  }
};
template <>
struct Mfma<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ float4 run(v8 a, v8 b, float4 c) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    f4 r = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, f4{c.x, c.y, c.z, c.w}, 0, 0, 0);
    return make_float4(r[0], r[1], r[2], r[3]);
  }
};

template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 as_v8(uint4 v) {
  typename Mfma<T>::v8 r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

struct DecodeArgs {
  const void *q;
  int64_t q_ss, q_hs;
  const void *kc, *vc;
  PoolView pool;
  const int32_t *bt;
  int32_t bt_stride;
  const int32_t *seq_lens;
  int32_t num_q_heads;
  float scale_log2;
  int32_t pages_per_split;
  int32_t max_splits;
  int32_t key_cap;  // keys any sequence may have: min(table width, splits * split size) * BS
  void *out;
  int64_t o_ss, o_hs;
  float *ws_m, *ws_l, *ws_acc;
  int32_t *counters;  // one per (sequence, KV head)
};

template <typename T, int DH, int G>
__global__ __launch_bounds__(64) void decode_mfma_kernel(DecodeArgs a) {
  constexpr int BS = 16;
  constexpr int NC = DH / 32;    // MFMA k-chunks of the QK product
  constexpr int LPR = DH / 2;    // lanes covering one V row, 2 dims each
  constexpr int HG = 64 / LPR;   // head groups across the wave
  constexpr int HPL = G / HG;    // heads accumulated per lane
  static_assert(DH == 64 || DH == 128, "head_dim");
  static_assert(G >= HG && G % HG == 0 && 16 % G == 0, "group size");
  __shared__ __attribute__((aligned(16))) float p_s[G][BS];
  __shared__ __attribute__((aligned(16))) float alpha_s[G];
  __shared__ __attribute__((aligned(16))) float l_s[G];

  const int lane = threadIdx.x;
  const int r = lane & 15;     // MFMA column: token within the page
  const int grp = lane >> 4;   // MFMA k-group / output row block
  const int pc = lane % LPR;   // dim pair owned in P.V
  const int hg = lane / LPR;   // head group owned in P.V

  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  // A length above the host bound is clamped so that no table, pool or workspace
  // access can leave its buffer.
  const int len = min(a.seq_lens[b], a.key_cap);
  const int n_pages = (len + BS - 1) / BS;
  const int p_begin = split * a.pages_per_split;
  const T *q = static_cast<const T *>(a.q);
  T *out = static_cast<T *>(a.out);

  if (p_begin >= n_pages) {
    if (split == 0) {  // empty sequence: defined all-zero output
#pragma unroll
      for (int j = 0; j < HPL; ++j) {
        T *op = out + b * a.o_ss + (int64_t)(kvh * G + hg * HPL + j) * a.o_hs + 2 * pc;
        op[0] = from_float<T>(0.f);
        op[1] = from_float<T>(0.f);
      }
    }
    return;
  }
  const int p_end = min(n_pages, p_begin + a.pages_per_split);

  // S^T tile: A = Q with row m <-> head m % G (replicated), B = K^T with column
  // n <-> token n, k-slot grp*8+j of chunk c <-> dim c*32 + grp*8 + j.
  // Lane (grp, r) receives rows grp*4+i, i.e. heads (grp*4+i) % G, for token r.
  typename Mfma<T>::v8 qa[NC];
  {
    const T *qp = q + b * a.q_ss + (int64_t)(kvh * G + r % G) * a.q_hs + grp * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) qa[c] = as_v8<T>(ld16(qp + c * 32));
  }

  const T *kc = static_cast<const T *>(a.kc);
  const T *vc = static_cast<const T *>(a.vc);
  const int64_t page_base = a.pool.layer_base + (int64_t)kvh * a.pool.head_stride;
  const int k_off = r * DH + grp * 8;  // + c*32
  const int v_off = 2 * pc;            // + t*DH
  const int32_t *bt_row = a.bt + (int64_t)b * a.bt_stride;

  float acc[HPL][2];
#pragma unroll
  for (int j = 0; j < HPL; ++j) acc[j][0] = acc[j][1] = 0.f;
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
  }

  uint4 kb[NC];
  uint32_t vb[BS];
  {
    const int64_t off = page_base + block_of(bt_row, p_begin, a.pool.num_blocks) * a.pool.block_stride;
#pragma unroll
    for (int c = 0; c < NC; ++c) kb[c] = ld16(kc + off + k_off + c * 32);
#pragma unroll
    for (int t = 0; t < BS; ++t)
      vb[t] = *reinterpret_cast<const uint32_t *>(vc + off + t * DH + v_off);
  }

  for (int p = p_begin; p < p_end; ++p) {
    uint4 kcur[NC];
    uint32_t vcur[BS];
#pragma unroll
    for (int c = 0; c < NC; ++c) kcur[c] = kb[c];
#pragma unroll
    for (int t = 0; t < BS; ++t) vcur[t] = vb[t];
    if (p + 1 < p_end) {  // prefetch the next page while this one is consumed
      const int64_t off = page_base + block_of(bt_row, p + 1, a.pool.num_blocks) * a.pool.block_stride;
#pragma unroll
      for (int c = 0; c < NC; ++c) kb[c] = ld16(kc + off + k_off + c * 32);
#pragma unroll
      for (int t = 0; t < BS; ++t)
        vb[t] = *reinterpret_cast<const uint32_t *>(vc + off + t * DH + v_off);
    }

    float4 s4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int c = 0; c < NC; ++c) s4 = Mfma<T>::run(qa[c], as_v8<T>(kcur[c]), s4);

    // Online softmax for the 4 heads this lane produces (token r).
    const bool valid = p * BS + r < len;
    const float s[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sv = valid ? s[i] * a.scale_log2 : -INFINITY;
      const float mn = fmaxf(m[i], row16_max(sv));
      const float alpha = exp2f(m[i] - mn);
      const float pv = exp2f(sv - mn);
      m[i] = mn;
      l[i] = l[i] * alpha + pv;
      const int h = grp * 4 + i;
      if (h < G) {
        p_s[h][r] = pv;
        if (r == 0) alpha_s[h] = alpha;
      }
    }
    __syncthreads();

    // P.V: lane owns dims (2pc, 2pc+1) of heads hg*HPL .. +HPL, all 16 tokens.
    float v0[BS], v1[BS];
#pragma unroll
    for (int t = 0; t < BS; ++t) {
      if constexpr (sizeof(T) == 2) {
        T lo, hi;
        const uint16_t wl = static_cast<uint16_t>(vcur[t] & 0xffffu);
        const uint16_t wh = static_cast<uint16_t>(vcur[t] >> 16);
        __builtin_memcpy(&lo, &wl, 2);
        __builtin_memcpy(&hi, &wh, 2);
        v0[t] = to_float(lo);
        v1[t] = to_float(hi);
      }
    }
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
      const int h = hg * HPL + j;
      const float al = alpha_s[h];
      float a0 = acc[j][0] * al, a1 = acc[j][1] * al;
#pragma unroll
      for (int t = 0; t < BS; t += 4) {
        const float4 pv = *reinterpret_cast<const float4 *>(&p_s[h][t]);
        a0 += pv.x * v0[t] + pv.y * v0[t + 1] + pv.z * v0[t + 2] + pv.w * v0[t + 3];
        a1 += pv.x * v1[t] + pv.y * v1[t + 1] + pv.z * v1[t + 2] + pv.w * v1[t + 3];
      }
      acc[j][0] = a0;
      acc[j][1] = a1;
    }
    __syncthreads();
  }

  // Softmax denominators: sum the producers' token partials over the 16 tokens.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    l[i] = row16_sum(l[i]);
    const int h = grp * 4 + i;
    if (h < G && r == 0) l_s[h] = l[i];
  }
  __syncthreads();

  const int n_splits = (n_pages + a.pages_per_split - 1) / a.pages_per_split;
  if (n_splits == 1) {
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
      const int h = hg * HPL + j;
      const float inv = 1.f / l_s[h];
      T *op = out + b * a.o_ss + (int64_t)(kvh * G + h) * a.o_hs + v_off;
      op[0] = from_float<T>(acc[j][0] * inv);
      op[1] = from_float<T>(acc[j][1] * inv);
    }
    return;
  }
  const int64_t w0 = ((int64_t)b * a.num_q_heads + kvh * G) * a.max_splits + split;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = grp * 4 + i;
    if (h < G && r == 0) {
      a.ws_m[w0 + (int64_t)h * a.max_splits] = m[i];
      a.ws_l[w0 + (int64_t)h * a.max_splits] = l[i];
    }
  }
#pragma unroll
  for (int j = 0; j < HPL; ++j) {
    const int h = hg * HPL + j;
    float *wp = a.ws_acc + (w0 + (int64_t)h * a.max_splits) * DH + v_off;
    wp[0] = acc[j][0];
    wp[1] = acc[j][1];
  }
  int32_t *counter = a.counters + (int64_t)b * gridDim.y + kvh;
  if (!arrive_last(counter, n_splits)) return;
#pragma unroll
  for (int j = 0; j < HPL; ++j) {
    const int h = hg * HPL + j;
    const int64_t w = ((int64_t)b * a.num_q_heads + kvh * G + h) * a.max_splits;
    float inv0, inv1;
    const float o0 = merge_splits(a.ws_m, a.ws_l, a.ws_acc, w, n_splits, DH, v_off, &inv0);
    const float o1 = merge_splits(a.ws_m, a.ws_l, a.ws_acc, w, n_splits, DH, v_off + 1, &inv1);
    T *op = out + b * a.o_ss + (int64_t)(kvh * G + h) * a.o_hs + v_off;
    op[0] = from_float<T>(o0 * inv0);
    op[1] = from_float<T>(o1 * inv1);
  }
  release_counter(counter);
}

// ------------------------------------------------------------------------
// Generic kernel (VALU), one wave per (row, KV head, split)
// ------------------------------------------------------------------------

constexpr int kGenMaxG = 16;
constexpr int kGenMaxDh = 128;
constexpr int kGenOut = kGenMaxG * kGenMaxDh / 64;  // outputs per lane

struct GenericArgs {
  const void *q;
  int64_t q_rs, q_hs;  // row (token or sequence) and head strides of the query
  const void *kc, *vc;
  PoolView pool;
  const int32_t *bt;
  int32_t bt_stride;
  const int32_t *seq_lens;
  const int32_t *cu_q;  // null: row == sequence (decode); else ragged prefill rows
  int32_t num_seqs;
  int32_t num_q_heads;
  int32_t group;  // G
  float scale_log2;
  int32_t pages_per_split;
  int32_t max_splits;
  int32_t key_cap;  // keys any row may have: min(table width, splits * split size) * BS
  void *out;
  int64_t o_rs, o_hs;
  float *ws_m, *ws_l, *ws_acc;
  int32_t *counters;  // one per (row, KV head)
};

template <typename T>
__global__ __launch_bounds__(64) void attn_generic_kernel(GenericArgs a) {
  __shared__ float q_s[kGenMaxG][kGenMaxDh];
  __shared__ float p_s[kGenMaxG][64];
  __shared__ int64_t row_s[64];

  const int lane = threadIdx.x;
  const int row = blockIdx.x / a.max_splits;
  const int split = blockIdx.x - row * a.max_splits;
  const int kvh = blockIdx.y;
  const int G = a.group;
  const int DH = a.pool.head_dim;
  const int BS = a.pool.block_size;

  int seq, kv_len;
  if (a.cu_q == nullptr) {
    seq = row;
    kv_len = a.seq_lens[row];
  } else {
    int lo = 0, hi = a.num_seqs;  // last seq with cu_q[seq] <= row
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (a.cu_q[mid] <= row) lo = mid; else hi = mid;
    }
    seq = lo;
    const int q_len = a.cu_q[seq + 1] - a.cu_q[seq];
    kv_len = a.seq_lens[seq] - q_len + (row - a.cu_q[seq]) + 1;
  }
  kv_len = min(kv_len, a.key_cap);
  const T *q = static_cast<const T *>(a.q);
  T *out = static_cast<T *>(a.out);
  const int tok_per_split = a.pages_per_split * BS;
  const int t_begin = split * tok_per_split;
  if (t_begin >= kv_len) {
    if (split == 0)
      for (int i = lane; i < G * DH; i += 64)
        out[(int64_t)row * a.o_rs + (int64_t)(kvh * G + i / DH) * a.o_hs + i % DH] =
            from_float<T>(0.f);
    return;
  }
  const int t_end = min(kv_len, t_begin + tok_per_split);

  for (int i = lane; i < G * DH; i += 64) {
    const int g = i / DH, d = i % DH;
    q_s[g][d] = to_float(q[(int64_t)row * a.q_rs + (int64_t)(kvh * G + g) * a.q_hs + d]);
  }

  float acc[kGenOut];
#pragma unroll
  for (int k = 0; k < kGenOut; ++k) acc[k] = 0.f;
  float m[kGenMaxG], l[kGenMaxG];
#pragma unroll
  for (int g = 0; g < kGenMaxG; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
  }
  const T *kc = static_cast<const T *>(a.kc);
  const T *vc = static_cast<const T *>(a.vc);
  const int32_t *bt_row = a.bt + (int64_t)seq * a.bt_stride;
  __syncthreads();

  for (int t0 = t_begin; t0 < t_end; t0 += 64) {
    const int t = t0 + lane;
    const bool valid = t < t_end;
    int64_t rb = 0;
    if (valid) {
      const int64_t blk = block_of(bt_row, t / BS, a.pool.num_blocks);
      rb = a.pool.layer_base + blk * a.pool.block_stride + (int64_t)kvh * a.pool.head_stride +
           (int64_t)(t % BS) * DH;
    }
    row_s[lane] = rb;
    float s[kGenMaxG];
#pragma unroll
    for (int g = 0; g < kGenMaxG; ++g) s[g] = 0.f;
    if (valid) {
      for (int d = 0; d < DH; ++d) {
        const float kv = to_float(kc[rb + d]);
#pragma unroll
        for (int g = 0; g < kGenMaxG; ++g)
          if (g < G) s[g] += q_s[g][d] * kv;
      }
    }
#pragma unroll
    for (int g = 0; g < kGenMaxG; ++g) {
      if (g < G) {
        const float sv = valid ? s[g] * a.scale_log2 : -INFINITY;
        const float mt = wave_max(sv);
        const float mn = fmaxf(m[g], mt);
        const float alpha = exp2f(m[g] - mn);
        const float pv = exp2f(sv - mn);
        l[g] = l[g] * alpha + wave_sum(pv);
        m[g] = mn;
        p_s[g][lane] = pv;
#pragma unroll
        for (int k = 0; k < kGenOut; ++k)
          if ((lane + 64 * k) / DH == g) acc[k] *= alpha;
      }
    }
    __syncthreads();
    const int n = min(64, t_end - t0);
    for (int j = 0; j < n; ++j) {
      const int64_t vb = row_s[j];
#pragma unroll
      for (int k = 0; k < kGenOut; ++k) {
        const int idx = lane + 64 * k;
        if (idx < G * DH) {
          const int g = idx / DH, d = idx % DH;
          acc[k] += p_s[g][j] * to_float(vc[vb + d]);
        }
      }
    }
    __syncthreads();
  }

  const int kv_pages = (kv_len + BS - 1) / BS;
  const int n_splits = (kv_pages + a.pages_per_split - 1) / a.pages_per_split;
#pragma unroll
  for (int k = 0; k < kGenOut; ++k) {
    const int idx = lane + 64 * k;
    if (idx >= G * DH) continue;
    const int g = idx / DH, d = idx % DH;
    const int qh = kvh * G + g;
    float lg = 0.f, mg = 0.f;
#pragma unroll
    for (int gg = 0; gg < kGenMaxG; ++gg)
      if (gg == g) {
        lg = l[gg];
        mg = m[gg];
      }
    if (n_splits == 1) {
      out[(int64_t)row * a.o_rs + (int64_t)qh * a.o_hs + d] = from_float<T>(acc[k] / lg);
    } else {
      const int64_t w = ((int64_t)row * a.num_q_heads + qh) * a.max_splits + split;
      if (d == 0) {
        a.ws_m[w] = mg;
        a.ws_l[w] = lg;
      }
      a.ws_acc[w * DH + d] = acc[k];
    }
  }
  if (n_splits == 1) return;
  int32_t *counter = a.counters + (int64_t)row * gridDim.y + kvh;
  if (!arrive_last(counter, n_splits)) return;
  for (int idx = lane; idx < G * DH; idx += 64) {
    const int g = idx / DH, d = idx % DH;
    const int qh = kvh * G + g;
    const int64_t w = ((int64_t)row * a.num_q_heads + qh) * a.max_splits;
    float inv;
    const float o = merge_splits(a.ws_m, a.ws_l, a.ws_acc, w, n_splits, DH, d, &inv);
    out[(int64_t)row * a.o_rs + (int64_t)qh * a.o_hs + d] = from_float<T>(o * inv);
  }
  release_counter(counter);
}

// ------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------

constexpr int kDefaultPages = 32;

int32_t choose_pages_per_split(int32_t num_seqs, int32_t num_kv_heads, int32_t block_size,
                               int32_t max_seq_len, int32_t requested) {
  if (requested > 0) return requested;
  const int64_t max_pages = ceil_div(max_seq_len > 0 ? max_seq_len : 1, block_size);
  // Aim for at least ~2048 work items (8 waves on each of 256 CUs); never split
  // below 8 pages, never above kDefaultPages.
  const int64_t items = static_cast<int64_t>(num_seqs) * num_kv_heads;
  int64_t pages = kDefaultPages;
  while (pages > 8 && items * ceil_div(max_pages, pages) < 2048) pages /= 2;
  return static_cast<int32_t>(pages);
}

struct Workspace {
  int32_t *counters;
  float *m, *l, *acc;
  int64_t bytes;
};

// Layout: [arrival counters, rows * Hkv int32][m][l][acc], each region 256-byte aligned.
Workspace carve(void *ws, int64_t rows, int32_t num_q_heads, int32_t num_kv_heads,
                int32_t max_splits, int32_t head_dim) {
  Workspace w;
  const int64_t nc = ceil_div(rows * num_kv_heads, 64) * 64;
  const int64_t n = rows * num_q_heads * max_splits;
  const int64_t n_al = ceil_div(n, 64) * 64;
  char *base = static_cast<char *>(ws);
  w.counters = reinterpret_cast<int32_t *>(base);
  w.m = base ? reinterpret_cast<float *>(base + nc * 4) : nullptr;
  w.l = base ? w.m + n_al : nullptr;
  w.acc = base ? w.l + n_al : nullptr;
  w.bytes = nc * 4 + (2 * n_al + n * head_dim) * static_cast<int64_t>(sizeof(float));
  return w;
}

bool pool_ok(int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
             int32_t head_dim) {
  return num_layers > 0 && num_blocks > 0 && num_kv_heads > 0 && block_size > 0 &&
         head_dim > 0 && head_dim <= kGenMaxDh;
}

PoolView make_pool(int32_t layer_index, int64_t num_blocks, int32_t num_kv_heads,
                   int32_t block_size, int32_t head_dim) {
  PoolView p;
  p.head_stride = static_cast<int64_t>(block_size) * head_dim;
  p.block_stride = p.head_stride * num_kv_heads;
  p.layer_base = p.block_stride * num_blocks * layer_index;
  p.num_blocks = num_blocks;
  p.block_size = block_size;
  p.head_dim = head_dim;
  return p;
}

template <typename T>
int32_t launch_decode_mfma(const DecodeArgs &a, int32_t num_seqs, int32_t num_kv_heads,
                           int32_t G, int32_t head_dim, hipStream_t s) {
  const dim3 grid(a.max_splits, num_kv_heads, num_seqs);
#define TKS_DECODE(DH, GG)                                     \
  if (head_dim == DH && G == GG) {                             \
    decode_mfma_kernel<T, DH, GG><<<grid, 64, 0, s>>>(a);      \
    return check_launch();                                     \
  }
  TKS_DECODE(128, 4)
  TKS_DECODE(128, 8)
  TKS_DECODE(128, 1)
  TKS_DECODE(128, 2)
  TKS_DECODE(128, 16)
  TKS_DECODE(64, 8)
  TKS_DECODE(64, 4)
  TKS_DECODE(64, 2)
  TKS_DECODE(64, 16)
#undef TKS_DECODE
  return TKS_ERR_VALUE;
}

template <typename T>
int32_t launch_generic(const GenericArgs &a, int32_t rows, int32_t num_kv_heads,
                       hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(rows) * a.max_splits),
                  num_kv_heads);
  attn_generic_kernel<T><<<grid, 64, 0, s>>>(a);
  return check_launch();
}

bool mfma_eligible(int32_t dtype, int32_t block_size, int32_t head_dim, int32_t G,
                   const void *q, int64_t q_ss, int64_t q_hs, const void *kc, const void *vc,
                   const void *out, int64_t o_ss, int64_t o_hs) {
  if (dtype == TKS_FLOAT32 || block_size != 16) return false;
  const bool shape = (head_dim == 128 && (G == 1 || G == 2 || G == 4 || G == 8 || G == 16)) ||
                     (head_dim == 64 && (G == 2 || G == 4 || G == 8 || G == 16));
  if (!shape) return false;
  return aligned16(q) && aligned16(kc) && aligned16(vc) && (reinterpret_cast<uintptr_t>(out) & 3u) == 0 &&
         q_ss % 8 == 0 && q_hs % 8 == 0 && o_ss % 2 == 0 && o_hs % 2 == 0;
}

}  // namespace
}  // namespace tks

using namespace tks;

extern "C" int64_t tks_paged_attention_decode_workspace_bytes(int32_t num_seqs,
                                                              int32_t num_q_heads,
                                                              int32_t num_kv_heads,
                                                              int32_t head_dim,
                                                              int32_t block_size,
                                                              int32_t max_seq_len,
                                                              int32_t pages_per_split) {
  if (num_seqs < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      block_size <= 0 || max_seq_len < 0 || pages_per_split < 0)
    return -1;
  const int32_t pps =
      choose_pages_per_split(num_seqs, num_kv_heads, block_size, max_seq_len, pages_per_split);
  const int32_t max_splits =
      static_cast<int32_t>(ceil_div(ceil_div(max_seq_len > 0 ? max_seq_len : 1, block_size), pps));
  if (max_splits <= 1) return 0;
  return carve(nullptr, num_seqs, num_q_heads, num_kv_heads, max_splits, head_dim).bytes;
}

extern "C" int32_t tks_paged_attention_decode(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, int32_t num_seqs, int32_t num_q_heads,
    int32_t max_seq_len, float scale, int32_t pages_per_split, void *out,
    int64_t out_seq_stride, int64_t out_head_stride, void *workspace, int64_t workspace_bytes,
    int32_t dtype, tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (!pool_ok(num_layers, num_blocks, num_kv_heads, block_size, head_dim) || num_seqs < 0 ||
      num_q_heads <= 0 || num_q_heads % num_kv_heads != 0 || max_seq_len < 0 ||
      pages_per_split < 0)
    return TKS_ERR_VALUE;
  const int32_t G = num_q_heads / num_kv_heads;
  if (G > kGenMaxG) return TKS_ERR_VALUE;
  if (layer_index < 0 || layer_index >= num_layers) return TKS_ERR_INDEX;
  if (num_seqs == 0) return TKS_OK;
  if (ceil_div(max_seq_len, block_size) > block_table_stride) return TKS_ERR_VALUE;
  if (!query || !key_cache || !value_cache || !block_tables || !seq_lens || !out)
    return TKS_ERR_VALUE;

  const int32_t pps =
      choose_pages_per_split(num_seqs, num_kv_heads, block_size, max_seq_len, pages_per_split);
  const int32_t max_splits =
      static_cast<int32_t>(ceil_div(ceil_div(max_seq_len > 0 ? max_seq_len : 1, block_size), pps));
  Workspace w = carve(workspace, num_seqs, num_q_heads, num_kv_heads, max_splits, head_dim);
  if (max_splits > 1 && (workspace == nullptr || workspace_bytes < w.bytes))
    return TKS_ERR_WORKSPACE;
  const int32_t key_cap = static_cast<int32_t>(
      std::min<int64_t>(block_table_stride, static_cast<int64_t>(max_splits) * pps) * block_size);

  const PoolView pool = make_pool(layer_index, num_blocks, num_kv_heads, block_size, head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float scale_log2 = scale * kLog2e;
  int32_t st;

  if (mfma_eligible(dtype, block_size, head_dim, G, query, q_seq_stride, q_head_stride,
                    key_cache, value_cache, out, out_seq_stride, out_head_stride)) {
    DecodeArgs a{query,        q_seq_stride,   q_head_stride, key_cache,      value_cache,
                 pool,         block_tables,   block_table_stride, seq_lens, num_q_heads,
                 scale_log2,   pps,            max_splits,    key_cap,        out,            out_seq_stride,
                 out_head_stride, w.m,         w.l,           w.acc,          w.counters};
    st = dtype == TKS_BFLOAT16
             ? launch_decode_mfma<bf16_t>(a, num_seqs, num_kv_heads, G, head_dim, s)
             : launch_decode_mfma<_Float16>(a, num_seqs, num_kv_heads, G, head_dim, s);
  } else {
    GenericArgs a{query,     q_seq_stride, q_head_stride, key_cache, value_cache, pool,
                  block_tables, block_table_stride, seq_lens, nullptr, num_seqs, num_q_heads,
                  G,         scale_log2,   pps,           max_splits, key_cap,    out,        out_seq_stride,
                  out_head_stride, w.m,    w.l,           w.acc,      w.counters};
    switch (dtype) {
      case TKS_FLOAT32: st = launch_generic<float>(a, num_seqs, num_kv_heads, s); break;
      case TKS_FLOAT16: st = launch_generic<_Float16>(a, num_seqs, num_kv_heads, s); break;
      default: st = launch_generic<bf16_t>(a, num_seqs, num_kv_heads, s); break;
    }
  }
  return st;
}

extern "C" int32_t tks_paged_attention_prefill(
    const void *query, int64_t q_token_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *cu_seqlens_q,
    int32_t num_seqs, int64_t num_tokens, int32_t num_q_heads, int32_t max_query_len,
    int32_t max_seq_len, float scale, void *out, int64_t out_token_stride,
    int64_t out_head_stride, int32_t dtype, tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (!pool_ok(num_layers, num_blocks, num_kv_heads, block_size, head_dim) || num_seqs < 0 ||
      num_tokens < 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      max_query_len < 0 || max_seq_len < 0 || max_query_len > max_seq_len)
    return TKS_ERR_VALUE;
  const int32_t G = num_q_heads / num_kv_heads;
  if (G > kGenMaxG) return TKS_ERR_VALUE;
  if (layer_index < 0 || layer_index >= num_layers) return TKS_ERR_INDEX;
  if (num_seqs == 0 || num_tokens == 0) return TKS_OK;
  if (num_tokens > 0x7fffffff) return TKS_ERR_VALUE;
  if (ceil_div(max_seq_len, block_size) > block_table_stride) return TKS_ERR_VALUE;
  if (!query || !key_cache || !value_cache || !block_tables || !seq_lens || !cu_seqlens_q ||
      !out)
    return TKS_ERR_VALUE;
  const PoolView pool = make_pool(layer_index, num_blocks, num_kv_heads, block_size, head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float scale_log2 = scale * kLog2e;
  // One split covering the whole key range: no partials, no workspace.
  const int32_t pps = static_cast<int32_t>(ceil_div(max_seq_len > 0 ? max_seq_len : 1, block_size));
  const int32_t key_cap = std::min(block_table_stride, pps) * block_size;
  GenericArgs a{query,     q_token_stride, q_head_stride, key_cache,  value_cache, pool,
                block_tables, block_table_stride, seq_lens, cu_seqlens_q, num_seqs, num_q_heads,
                G,         scale_log2,     pps,           1,          key_cap,     out,         out_token_stride,
                out_head_stride, nullptr,  nullptr,       nullptr,    nullptr};
  const int32_t rows = static_cast<int32_t>(num_tokens);
  switch (dtype) {
    case TKS_FLOAT32: return launch_generic<float>(a, rows, num_kv_heads, s);
    case TKS_FLOAT16: return launch_generic<_Float16>(a, rows, num_kv_heads, s);
    default: return launch_generic<bf16_t>(a, rows, num_kv_heads, s);
  }
}
