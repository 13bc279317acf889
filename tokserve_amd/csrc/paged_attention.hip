// Paged attention over block tables: host entry points and the generic kernel.
//
// Semantics follow tokserve/kernels/_triton_paged_attention.py:12-149: K/V are
// read through block_table[logical_block] (:76-82) from one layer of the
// [L, NB, Hkv, BS, Dh] pools, query head hq uses KV head hq / G (:49), the
// causal mask is key <= query position (:118-123), softmax is accumulated
// online in fp32 (:125-136) and the output is acc / sum in the query dtype (:138).
//
// Decode (one query per sequence) goes to decode_pv_kernel (decode_mfma.hip)
// for bf16/fp16 with block size 16 and Dh 64/128; every other shape and fp32
// (where 1e-5 parity wants fp32 products) uses attn_generic_kernel below:
// one 4-wave workgroup per (query row, KV head, split), 64 keys per wave step
// on the VALU. The
// generic kernel is also the ragged chunked-prefill path (one row per query
// token, causal key length).
//
// A decode batch with fewer (sequence, KV head) pairs than it takes to fill the
// GPU is also split across workgroups along the keys; the split partials
// (m, l, acc) then go to the caller's workspace and merge_splits_kernel, a
// second launch, combines them. Large batches run as one launch.
#include "attention_common.hpp"

#include <algorithm>
#include <atomic>
#include <mutex>

// Split-K partials of tks_paged_attention_decode_noalloc, for callers that may
// not allocate (code under HIP graph capture, serving loops that forbid
// allocation). Every GPU the library runs on holds its own copy until the
// process ends. Host code never uses this name as an address: the device
// address of each GPU's copy comes from hipGetSymbolAddress (scratch_address).
constexpr int64_t kStaticScratchBytes = int64_t{32} << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace tks {
namespace {

// ------------------------------------------------------------------------
// Generic kernel (VALU), one 4-wave workgroup per (row, KV head, split)
// ------------------------------------------------------------------------

constexpr int kGenMaxG = 16;
constexpr int kGenMaxDh = 128;
constexpr int kGenWaves = 4;
constexpr int kGenThreads = 64 * kGenWaves;

struct GenericArgs {
  const void *q;
  int64_t q_rs, q_hs;  // row (token or sequence) and head strides of the query
  const void *kc, *vc;
  PoolView pool;
  const int32_t *bt;
  int32_t bt_stride;
  const int32_t *seq_lens;
  const int32_t *seq_order;  // decode: workgroup slot -> sequence (null: identity)
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
  int32_t vec_rows;  // K/V rows are 16-byte aligned and head_dim is a multiple of 16 bytes
  float v_scale = 1.f;  // V decode factor of fp8 pools (1 otherwise)
  // fp8 pools with one scale per pool row ([L, NB, Hkv, BS], the pool row's element
  // offset / head_dim); null: per-pool scales.
  const float *k_rs = nullptr, *v_rs = nullptr;
};

// The split's keys are dealt to the four waves 64 at a time (wave w takes keys
// t_begin + 64 w + 256 i). In a step, lane t scores key t0 + t against the G
// query heads, and every K and V element the step needs is requested before
// the first is used, so a step costs about one memory latency. For P.V lane d
// accumulates dims d and d + 64 of all G heads; token j's row offset and
// probabilities are written to LDS by lane j and read back by all lanes as
// broadcasts (cheaper than a readlane, whose SGPR result stalls the next VALU
// use). Lanes past the valid range keep
// a zero row offset (an in-bounds read whose score is masked and whose V is
// zeroed). The waves' (m, l, acc) are combined through LDS at the end.
// DHMAX (64 or 128) bounds head_dim; dims past head_dim are zero in q and K.
template <typename T, typename KV, int DHMAX>
__global__ __launch_bounds__(kGenThreads) void attn_generic_kernel(GenericArgs a) {
  constexpr int V = Vec<KV>::N;
  constexpr int DPL = DHMAX / 64;  // dims per lane in P.V
  __shared__ __align__(16) float q_s[kGenMaxG][DHMAX];
  __shared__ float part_m[kGenWaves][kGenMaxG];
  __shared__ float part_l[kGenWaves][kGenMaxG];
  __shared__ __align__(16) float part_acc[kGenWaves][kGenMaxG][DHMAX];
  __shared__ __align__(16) int64_t rb_s[kGenWaves][64];  // a wave's row offsets, read back as broadcasts
  __shared__ __align__(16) float p_s[kGenWaves][kGenMaxG][64];  // a wave's probabilities, likewise

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int slot = blockIdx.x;
  const int split = blockIdx.z;
  const int row = a.seq_order ? min(max(a.seq_order[slot], 0), a.num_seqs - 1) : slot;
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
      for (int i = tid; i < G * DH; i += kGenThreads)
        out[(int64_t)row * a.o_rs + (int64_t)(kvh * G + i / DH) * a.o_hs + i % DH] =
            from_float<T>(0.f);
    return;
  }
  const int t_end = min(kv_len, t_begin + tok_per_split);

  const KV *kc = static_cast<const KV *>(a.kc);
  const KV *vc = static_cast<const KV *>(a.vc);
  const int32_t *bt_row = a.bt + (int64_t)seq * a.bt_stride;

  // Row offset of key t0 + lane (0 past the step's range) and the step's K row
  // and V columns; the first step is requested before q is staged.
  auto row_offset = [&](int t0) -> int64_t {
    const int t = t0 + lane;
    if (t >= t_end) return 0;
    const int64_t blk = block_of(bt_row, t / BS, a.pool.num_blocks);
    return a.pool.layer_base + blk * a.pool.block_stride + (int64_t)kvh * a.pool.head_stride +
           (int64_t)(t % BS) * DH;
  };
  float kv[DHMAX];
  float vv[64][DPL];
  // Row scales of this lane's key (scores) and value (probabilities); 1 and 1 for
  // per-pool scales. A lane past the step's keys reads row 0's and is masked.
  const bool rows = a.k_rs != nullptr;
  float ks_lane = 1.f, vs_lane = 1.f;
  auto load_step = [&](int64_t rb, int n) {
    if (rows) {
      ks_lane = a.k_rs[rb / DH];
      vs_lane = lane < n ? a.v_rs[rb / DH] : 0.f;
    }
    if (a.vec_rows) {
#pragma unroll
      for (int d = 0; d < DHMAX; d += V) {
        if (d < DH) {
          unpack<KV>(ld16(kc + rb + d), kv + d);
        } else {
#pragma unroll
          for (int i = 0; i < V; ++i) kv[d + i] = 0.f;
        }
      }
    } else {
#pragma unroll
      for (int d = 0; d < DHMAX; ++d) kv[d] = d < DH ? to_float(kc[rb + d]) : 0.f;
    }
    // LDS operations of one wave complete in order: the broadcast reads below
    // see this write without a barrier.
    rb_s[wave][lane] = rb;
#pragma unroll
    for (int u = 0; u < 64; ++u) {
      const int64_t vb = rb_s[wave][u];
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        const int d = lane + 64 * i;
        const float x = d < DH ? to_float(vc[vb + d]) : 0.f;
        vv[u][i] = u < n ? x : 0.f;
      }
    }
  };
  int t0 = t_begin + 64 * wave;
  if (t0 < t_end) load_step(row_offset(t0), min(64, t_end - t0));

  for (int i = tid; i < G * DHMAX; i += kGenThreads) {
    const int g = i / DHMAX, d = i % DHMAX;
    q_s[g][d] = d < DH ? to_float(q[(int64_t)row * a.q_rs + (int64_t)(kvh * G + g) * a.q_hs + d])
                       : 0.f;
  }

  float acc[kGenMaxG][DPL];
  float m[kGenMaxG], l[kGenMaxG];
#pragma unroll
  for (int g = 0; g < kGenMaxG; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[g][i] = 0.f;
  }
  __syncthreads();

  for (; t0 < t_end; t0 += 64 * kGenWaves) {
    const bool valid = t0 + lane < t_end;
    // q_s is loop-invariant: an opaque zero offset keeps its (broadcast) reads
    // inside the step instead of hoisted into G * DHMAX registers.
    int q_off = 0;
    asm volatile("" : "+v"(q_off));
    const float4 *qrow = reinterpret_cast<const float4 *>(&q_s[0][0]) + q_off;
    float pv[kGenMaxG];
#pragma unroll
    for (int g = 0; g < kGenMaxG; ++g) {
      pv[g] = 0.f;
      if (g < G) {
        float s = 0.f;
#pragma unroll
        for (int d = 0; d < DHMAX; d += 4) {
          const float4 qd = qrow[(g * DHMAX + d) / 4];
          s += qd.x * kv[d];
          s += qd.y * kv[d + 1];
          s += qd.z * kv[d + 2];
          s += qd.w * kv[d + 3];
        }
        const float sv = valid ? s * a.scale_log2 * ks_lane : -INFINITY;
        const float mt = wave_max(sv);
        const float mn = fmaxf(m[g], mt);
        const float alpha = fast_exp2(m[g] - mn);
        pv[g] = fast_exp2(sv - mn);
        l[g] = l[g] * alpha + wave_sum(pv[g]);
        m[g] = mn;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[g][i] *= alpha;
      }
    }
#pragma unroll
    for (int g = 0; g < kGenMaxG; ++g)
      if (g < G) p_s[wave][g][lane] = rows ? pv[g] * vs_lane : pv[g];
#pragma unroll
    for (int g = 0; g < kGenMaxG; ++g)
      if (g < G) {
#pragma unroll
        for (int u = 0; u < 64; ++u) {
          const float p = p_s[wave][g][u];
#pragma unroll
          for (int i = 0; i < DPL; ++i) acc[g][i] += p * vv[u][i];
        }
      }
    const int t_next = t0 + 64 * kGenWaves;
    if (t_next < t_end) load_step(row_offset(t_next), min(64, t_end - t_next));
  }

#pragma unroll
  for (int g = 0; g < kGenMaxG; ++g)
    if (g < G) {
      if (lane == 0) {
        part_m[wave][g] = m[g];
        part_l[wave][g] = l[g];
      }
#pragma unroll
      for (int i = 0; i < DPL; ++i) part_acc[wave][g][lane + 64 * i] = acc[g][i];
    }
  __syncthreads();
  // Wave 0 always has keys, so the maximum is finite for finite scores and a
  // wave without keys (m = -inf, l = 0, acc = 0) contributes nothing.
  for (int i = tid; i < G * DH; i += kGenThreads) {
    const int g = i / DH, d = i % DH;
    float mx = part_m[0][g];
#pragma unroll
    for (int w = 1; w < kGenWaves; ++w) mx = fmaxf(mx, part_m[w][g]);
    float lsum = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kGenWaves; ++w) {
      const float f = fast_exp2(part_m[w][g] - mx);
      lsum += part_l[w][g] * f;
      o += part_acc[w][g][d] * f;
    }
    const int qh = kvh * G + g;
    if (a.max_splits == 1) {
      out[(int64_t)row * a.o_rs + (int64_t)qh * a.o_hs + d] =
          from_float<T>(o / lsum * a.v_scale);
    } else {
      const int64_t w = ((int64_t)row * a.num_q_heads + qh) * a.max_splits + split;
      if (d == 0) {
        a.ws_m[w] = mx;
        a.ws_l[w] = lsum;
      }
      a.ws_acc[w * DH + d] = o * a.v_scale;
    }
  }
}

// ------------------------------------------------------------------------
// fp8 pools under the MFMA prefill: the pages a batch reads are decoded once
// into a dense scratch pool, page (b, p) at block b * W + p (W = the table
// width), with the identity table beside it. The scales are not applied here
// (k_scale rides on the score scale, v_scale on the output), so the scratch
// holds the exact e4m3 values in T.
// ------------------------------------------------------------------------

struct ScratchPages {
  void *k, *v;
  int32_t *table;
  int64_t bytes;
};

ScratchPages carve_pages(void *ws, int32_t num_seqs, int32_t table_width, int32_t num_kv_heads,
                         int32_t block_size, int32_t head_dim) {
  const int64_t pages = static_cast<int64_t>(num_seqs) * table_width;
  const int64_t pool = ceil_div(pages * num_kv_heads * block_size * head_dim * 2, 256) * 256;
  const int64_t table = ceil_div(pages * 4, 256) * 256;
  char *base = static_cast<char *>(ws);
  ScratchPages s;
  s.k = base;
  s.v = base ? base + pool : nullptr;
  s.table = base ? reinterpret_cast<int32_t *>(base + 2 * pool) : nullptr;
  s.bytes = 2 * pool + table;
  return s;
}

template <typename T>
__global__ __launch_bounds__(256) void decode_pages_kernel(
    const fp8e4m3_t *__restrict__ kc, const fp8e4m3_t *__restrict__ vc, PoolView pool,
    int32_t num_kv_heads, const int32_t *__restrict__ bt, int32_t bt_stride,
    const int32_t *__restrict__ seq_lens, int32_t num_seqs, T *__restrict__ k_out,
    T *__restrict__ v_out, int32_t *__restrict__ table_out, const float *__restrict__ k_rs,
    const float *__restrict__ v_rs) {
  const int64_t chunks = static_cast<int64_t>(pool.block_size) * pool.head_dim / 16;
  const int64_t per_page = chunks * num_kv_heads;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t slot = item / per_page;  // b * W + p
  if (slot >= static_cast<int64_t>(num_seqs) * bt_stride) return;
  const int b = static_cast<int>(slot / bt_stride);
  const int p = static_cast<int>(slot - static_cast<int64_t>(b) * bt_stride);
  const int64_t rem = item - slot * per_page;
  const int h = static_cast<int>(rem / chunks);
  const int64_t c = (rem - h * chunks) * 16;
  if (rem == 0) table_out[slot] = static_cast<int32_t>(slot);
  const int64_t len = min(static_cast<int64_t>(max(seq_lens[b], 0)),
                          static_cast<int64_t>(bt_stride) * pool.block_size);
  if (p * static_cast<int64_t>(pool.block_size) >= len) return;
  const int64_t blk = block_of(bt + static_cast<int64_t>(b) * bt_stride, p, pool.num_blocks);
  const int64_t src = pool.layer_base + blk * pool.block_stride + h * pool.head_stride + c;
  const int64_t dst = slot * pool.block_stride + h * pool.head_stride + c;
  float f[16];
  constexpr int N = Vec<T>::N;
  // Row scales (one per 16-element chunk's row: head_dim is a multiple of 16).
  const float ks = k_rs ? k_rs[src / pool.head_dim] : 1.f;
  const float vs = v_rs ? v_rs[src / pool.head_dim] : 1.f;
  unpack<fp8e4m3_t>(ld16(kc + src), f);
  if (k_rs) {
#pragma unroll
    for (int i = 0; i < 16; ++i) f[i] *= ks;
  }
#pragma unroll
  for (int i = 0; i < 16; i += N) st16(k_out + dst + i, pack<T>(f + i));
  unpack<fp8e4m3_t>(ld16(vc + src), f);
  if (v_rs) {
#pragma unroll
    for (int i = 0; i < 16; ++i) f[i] *= vs;
  }
#pragma unroll
  for (int i = 0; i < 16; i += N) st16(v_out + dst + i, pack<T>(f + i));
}

// ------------------------------------------------------------------------
// Split merge (second launch, only when a cross-workgroup split exists)
// ------------------------------------------------------------------------

template <typename T>
__global__ __launch_bounds__(128) void merge_splits_kernel(
    const int32_t *__restrict__ seq_lens, int32_t key_cap, int32_t block_size,
    int32_t pages_per_split, int32_t max_splits, int32_t num_q_heads, int32_t head_dim,
    const float *__restrict__ ws_m, const float *__restrict__ ws_l,
    const float *__restrict__ ws_acc, T *out, int64_t o_rs, int64_t o_hs) {
  const int qh = blockIdx.x;
  const int row = blockIdx.y;
  const int len = min(seq_lens[row], key_cap);
  const int n_pages = (len + block_size - 1) / block_size;
  const int n_splits = min((n_pages + pages_per_split - 1) / pages_per_split, max_splits);
  if (n_splits == 0) return;  // the split kernel wrote the zero row
  const int64_t w = ((int64_t)row * num_q_heads + qh) * max_splits;
  for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
    float inv;
    const float o = merge_splits(ws_m, ws_l, ws_acc, w, n_splits, head_dim, d, &inv);
    out[row * o_rs + (int64_t)qh * o_hs + d] = from_float<T>(o * inv);
  }
}

// ------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------

// Key splits for decode. A (sequence, KV head) pair runs as one workgroup
// whose four waves walk its pages in order, so an unsplit launch lasts at least
// as long as its longest sequence takes; with few pairs that chain, not the
// bytes, sets the time. Splits are merged by a second launch.
//  * Fewer than kFillItems pairs (less than one workgroup per CU): cut every
//    sequence so the batch has about kFillItems workgroups, splits of 16 to 48
//    pages (fp32 decode step, 8 sequences x 2 KV heads, contexts <= 513: 12.8 +
//    4.0 us merge split against 18.4 us unsplit; 8 / 16 Llama-3-8B sequences x 8
//    KV heads, contexts log-uniform in [128, 8192]: 39.3 / 41.8 us at 64 pages,
//    34.8 / 37.0 us at 48, 39.3 / 45.9 us at 16; 16 sequences unsplit: 59 us).
//  * Fewer than kSplitBelowItems pairs and a length bound of kSplitFromPages
//    pages or more: 32-page splits (32 / 64 such Llama-3-8B sequences with the
//    MFMA P.V kernel, split and merge: 45.3 / 90.5 us at 32 pages, 47.6 / 91.2 at
//    64, 74.1 / 110.7 unsplit).
//  * Otherwise unsplit: 128, 192 and 256 Llama-3-8B sequences (128: 161.4 us
//    against 166.2 at 64 pages and 173.3 at 32; 192: 216.4 against 249.6+ split),
//    and short contexts (128 sequences x 4 KV heads, Dh 64, contexts up to 1152
//    under a 2048-token bound).
constexpr int64_t kFillItems = 256;
constexpr int64_t kMinSplitPages = 16;
constexpr int64_t kMaxFillSplitPages = 48;
constexpr int64_t kSplitBelowItems = 1024;
constexpr int64_t kSplitPages = 32;
constexpr int64_t kSplitFromPages = 256;

int32_t choose_pages_per_split(int32_t num_seqs, int32_t num_kv_heads, int32_t block_size,
                               int32_t max_seq_len, int32_t requested) {
  if (requested > 0) return requested;
  const int64_t max_pages = ceil_div(max_seq_len > 0 ? max_seq_len : 1, block_size);
  const int64_t items = static_cast<int64_t>(num_seqs) * num_kv_heads;
  if (items > 0 && items < kFillItems) {
    const int64_t per_split = ceil_div(max_pages, ceil_div(kFillItems, items));
    return static_cast<int32_t>(std::min(kMaxFillSplitPages, std::max(kMinSplitPages, per_split)));
  }
  if (items < kSplitBelowItems && max_pages >= kSplitFromPages)
    return static_cast<int32_t>(kSplitPages);
  return static_cast<int32_t>(max_pages);
}

int32_t split_count(int32_t max_seq_len, int32_t block_size, int32_t pps) {
  return static_cast<int32_t>(ceil_div(ceil_div(max_seq_len > 0 ? max_seq_len : 1, block_size), pps));
}

struct Workspace {
  float *m, *l, *acc;
  int64_t bytes;
};

// Layout: [m][l][acc] per (row, q head, split), m and l padded to 64 entries.
Workspace carve(void *ws, int64_t rows, int32_t num_q_heads, int32_t max_splits,
                int32_t head_dim) {
  Workspace w;
  const int64_t n = rows * num_q_heads * max_splits;
  const int64_t n_al = ceil_div(n, 64) * 64;
  w.m = static_cast<float *>(ws);
  w.l = ws ? w.m + n_al : nullptr;
  w.acc = ws ? w.l + n_al : nullptr;
  w.bytes = (2 * n_al + n * head_dim) * static_cast<int64_t>(sizeof(float));
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

template <typename T, typename KV>
int32_t launch_generic_kv(const GenericArgs &a, int32_t rows, int32_t num_kv_heads,
                          hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(rows), num_kv_heads, a.max_splits);
  if (a.pool.head_dim <= 64)
    attn_generic_kernel<T, KV, 64><<<grid, kGenThreads, 0, s>>>(a);
  else
    attn_generic_kernel<T, KV, 128><<<grid, kGenThreads, 0, s>>>(a);
  return check_launch();
}

int32_t launch_generic(const GenericArgs &a, int32_t dtype, int32_t rows, int32_t num_kv_heads,
                       bool fp8_pools, hipStream_t s) {
  switch (dtype) {
    case TKS_FLOAT32:
      return fp8_pools ? launch_generic_kv<float, fp8e4m3_t>(a, rows, num_kv_heads, s)
                       : launch_generic_kv<float, float>(a, rows, num_kv_heads, s);
    case TKS_FLOAT16:
      return fp8_pools ? launch_generic_kv<_Float16, fp8e4m3_t>(a, rows, num_kv_heads, s)
                       : launch_generic_kv<_Float16, _Float16>(a, rows, num_kv_heads, s);
    default:
      return fp8_pools ? launch_generic_kv<bf16_t, fp8e4m3_t>(a, rows, num_kv_heads, s)
                       : launch_generic_kv<bf16_t, bf16_t>(a, rows, num_kv_heads, s);
  }
}

// K/V rows can be read 16 bytes at a time: pools aligned, rows a multiple of 16 bytes.
int32_t vec_rows_ok(const void *kc, const void *vc, int32_t head_dim, int elem) {
  return aligned16(kc) && aligned16(vc) && (head_dim * elem) % 16 == 0;
}

bool mfma_eligible(int32_t dtype, int32_t block_size, int32_t head_dim, int32_t G,
                   const void *q, int64_t q_ss, int64_t q_hs, const void *kc, const void *vc,
                   const void *out, int64_t o_ss, int64_t o_hs) {
  if (block_size != 16 || !decode_mfma_supported(dtype, head_dim, G)) return false;
  return aligned16(q) && aligned16(kc) && aligned16(vc) && aligned16(out) && q_ss % 8 == 0 &&
         q_hs % 8 == 0 && o_ss % 8 == 0 && o_hs % 8 == 0;
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
  const int32_t max_splits = split_count(max_seq_len, block_size, pps);
  if (max_splits <= 1) return 0;
  return carve(nullptr, num_seqs, num_q_heads, max_splits, head_dim).bytes;
}

namespace {

// RoPE and the KV append of each sequence's new token, fused into a decode launch
// (tks_rope_append_paged_decode).
struct RopeAppend {
  const void *key;
  int64_t k_ss, k_hs;
  const void *value;
  int64_t v_ss, v_hs;
  const int64_t *positions;
  const void *cos_cache, *sin_cache;
  int64_t cache_len;
  const int64_t *slot_mapping;
};

int32_t decode_impl(const void *query, int64_t q_seq_stride, int64_t q_head_stride,
                    const void *key_cache, const void *value_cache, int32_t num_layers,
                    int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
                    int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
                    int32_t block_table_stride, const int32_t *seq_lens,
                    const int32_t *seq_order, int32_t num_seqs, int32_t num_q_heads,
                    int32_t max_seq_len, float scale, int32_t pages_per_split, void *out,
                    int64_t out_seq_stride, int64_t out_head_stride, void *workspace,
                    int64_t workspace_bytes, bool fp8_pools, float k_scale, float v_scale,
                    int32_t dtype, tks_stream_t stream, const RopeAppend *ra = nullptr,
                    const float *k_rs = nullptr, const float *v_rs = nullptr) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if ((k_rs != nullptr) != (v_rs != nullptr) || (k_rs != nullptr && !fp8_pools))
    return TKS_ERR_VALUE;
  if (!pool_ok(num_layers, num_blocks, num_kv_heads, block_size, head_dim) || num_seqs < 0 ||
      num_q_heads <= 0 || num_q_heads % num_kv_heads != 0 || max_seq_len < 0 ||
      pages_per_split < 0 || !valid_scale(k_scale) || !valid_scale(v_scale))
    return TKS_ERR_VALUE;
  const int32_t G = num_q_heads / num_kv_heads;
  if (G > kGenMaxG) return TKS_ERR_VALUE;
  if (layer_index < 0 || layer_index >= num_layers) return TKS_ERR_INDEX;
  if (num_seqs == 0) return TKS_OK;
  if (num_seqs > 65535 || ceil_div(max_seq_len, block_size) > block_table_stride)
    return TKS_ERR_VALUE;
  if (!query || !key_cache || !value_cache || !block_tables || !seq_lens || !out)
    return TKS_ERR_VALUE;

  const int32_t pps =
      choose_pages_per_split(num_seqs, num_kv_heads, block_size, max_seq_len, pages_per_split);
  const int32_t max_splits = split_count(max_seq_len, block_size, pps);
  if (max_splits > kMaxGridSplits) return TKS_ERR_VALUE;
  Workspace w = carve(workspace, num_seqs, num_q_heads, max_splits, head_dim);
  if (max_splits > 1 && (workspace == nullptr || workspace_bytes < w.bytes))
    return TKS_ERR_WORKSPACE;
  const int32_t key_cap = static_cast<int32_t>(
      std::min<int64_t>(block_table_stride, static_cast<int64_t>(max_splits) * pps) * block_size);

  const PoolView pool = make_pool(layer_index, num_blocks, num_kv_heads, block_size, head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float scale_log2 = scale * kLog2e * k_scale;

  const bool mfma = mfma_eligible(dtype, block_size, head_dim, G, query, q_seq_stride,
                                  q_head_stride, key_cache, value_cache, out, out_seq_stride,
                                  out_head_stride);
  if (ra != nullptr) {
    // Fused when the MFMA kernel runs with its new rows in 16-byte chunks; otherwise
    // the RoPE + append launch writes the rotated queries into `out`, which the
    // decode then reads as its query (each workgroup reads its rows before it, or
    // the merge, writes them).
    const bool fused = mfma && aligned16(ra->key) && aligned16(ra->value) &&
                       aligned16(ra->cos_cache) && aligned16(ra->sin_cache) && ra->k_ss % 8 == 0 && ra->k_hs % 8 == 0 &&
                       ra->v_ss % 8 == 0 && ra->v_hs % 8 == 0;
    if (!fused) {
      void *kc = const_cast<void *>(key_cache), *vc = const_cast<void *>(value_cache);
      const int32_t st0 =
          k_rs != nullptr
              ? tks_rope_kv_append_fp8_rows(
                    query, out, q_seq_stride, q_head_stride, out_seq_stride, out_head_stride,
                    num_q_heads, ra->key, nullptr, ra->k_ss, ra->k_hs, 0, 0, ra->value,
                    ra->v_ss, ra->v_hs, num_kv_heads, num_seqs, head_dim, ra->positions,
                    ra->cos_cache, ra->sin_cache, ra->cache_len, kc, vc,
                    const_cast<float *>(k_rs), const_cast<float *>(v_rs), num_layers,
                    num_blocks, block_size, layer_index, ra->slot_mapping, dtype, stream)
          : fp8_pools
              ? tks_rope_kv_append_fp8(query, out, q_seq_stride, q_head_stride, out_seq_stride,
                                       out_head_stride, num_q_heads, ra->key, nullptr, ra->k_ss,
                                       ra->k_hs, 0, 0, ra->value, ra->v_ss, ra->v_hs,
                                       num_kv_heads, num_seqs, head_dim, ra->positions,
                                       ra->cos_cache, ra->sin_cache, ra->cache_len, kc, vc,
                                       num_layers, num_blocks, block_size, layer_index,
                                       ra->slot_mapping, k_scale, v_scale, dtype, stream)
              : tks_rope_kv_append(query, out, q_seq_stride, q_head_stride, out_seq_stride,
                                   out_head_stride, num_q_heads, ra->key, nullptr, ra->k_ss,
                                   ra->k_hs, 0, 0, ra->value, ra->v_ss, ra->v_hs, num_kv_heads,
                                   num_seqs, head_dim, ra->positions, ra->cos_cache,
                                   ra->sin_cache, ra->cache_len, kc, vc, num_layers, num_blocks,
                                   block_size, layer_index, ra->slot_mapping, dtype, stream);
      if (st0 != TKS_OK) return st0;
      return decode_impl(out, out_seq_stride, out_head_stride, key_cache, value_cache,
                         num_layers, num_blocks, num_kv_heads, block_size, head_dim, layer_index,
                         block_tables, block_table_stride, seq_lens, seq_order, num_seqs,
                         num_q_heads, max_seq_len, scale, pages_per_split, out, out_seq_stride,
                         out_head_stride, workspace, workspace_bytes, fp8_pools, k_scale, v_scale,
                         dtype, stream, nullptr, k_rs, v_rs);
    }
  }

  int32_t st;
  if (mfma) {
    DecodeArgs a{query,      q_seq_stride, q_head_stride, key_cache,   value_cache,
                 pool,       block_tables, block_table_stride, seq_lens, seq_order, num_q_heads,
                 scale_log2, pps,          max_splits,    key_cap,     out,
                 out_seq_stride, out_head_stride, w.m,    w.l,         w.acc,
                 v_scale};
    a.k_rs = k_rs;
    a.v_rs = v_rs;
    if (ra != nullptr) {
      a.positions = ra->positions;
      a.cos_t = ra->cos_cache;
      a.sin_t = ra->sin_cache;
      a.table_len = ra->cache_len;
      a.k_new = ra->key;
      a.kn_ss = ra->k_ss;
      a.kn_hs = ra->k_hs;
      a.v_new = ra->value;
      a.vn_ss = ra->v_ss;
      a.vn_hs = ra->v_hs;
      a.slots = ra->slot_mapping;
      a.k_scale = k_scale;
    }
    st = launch_decode_mfma(a, dtype, num_seqs, num_kv_heads, G, head_dim, s, fp8_pools);
  } else {
    const int kv_elem = fp8_pools ? 1 : elem_bytes(dtype);
    GenericArgs a{query,     q_seq_stride, q_head_stride, key_cache, value_cache, pool,
                  block_tables, block_table_stride, seq_lens, seq_order, nullptr, num_seqs, num_q_heads,
                  G,         scale_log2,   pps,           max_splits, key_cap,  out,
                  out_seq_stride, out_head_stride, w.m,   w.l,        w.acc,
                  vec_rows_ok(key_cache, value_cache, head_dim, kv_elem), v_scale};
    a.k_rs = k_rs;
    a.v_rs = v_rs;
    st = launch_generic(a, dtype, num_seqs, num_kv_heads, fp8_pools, s);
  }
  if (st != TKS_OK || max_splits == 1) return st;
  const dim3 grid(num_q_heads, num_seqs);
  const int threads = head_dim > 64 ? 128 : 64;  // one thread per output element
#define TKS_MERGE(TYPE)                                                                         \
  merge_splits_kernel<TYPE><<<grid, threads, 0, s>>>(seq_lens, key_cap, block_size, pps,        \
                                                     max_splits, num_q_heads, head_dim, w.m, w.l, \
                                                     w.acc, static_cast<TYPE *>(out),             \
                                                     out_seq_stride, out_head_stride)
  switch (dtype) {
    case TKS_FLOAT32: TKS_MERGE(float); break;
    case TKS_FLOAT16: TKS_MERGE(_Float16); break;
    default: TKS_MERGE(bf16_t); break;
  }
#undef TKS_MERGE
  return check_launch();
}

int32_t prefill_impl(const void *query, int64_t q_token_stride, int64_t q_head_stride,
                     const void *key_cache, const void *value_cache, int32_t num_layers,
                     int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
                     int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
                     int32_t block_table_stride, const int32_t *seq_lens,
                     const int32_t *cu_seqlens_q, const int32_t *seq_order, int32_t num_seqs,
                     int64_t num_tokens, int32_t num_q_heads, int32_t max_query_len,
                     int32_t max_seq_len, float scale, void *out, int64_t out_token_stride,
                     int64_t out_head_stride, bool fp8_pools, void *workspace,
                     int64_t workspace_bytes, float k_scale, float v_scale, int32_t dtype,
                     tks_stream_t stream, const float *k_rs = nullptr,
                     const float *v_rs = nullptr) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if ((k_rs != nullptr) != (v_rs != nullptr) || (k_rs != nullptr && !fp8_pools))
    return TKS_ERR_VALUE;
  if (!pool_ok(num_layers, num_blocks, num_kv_heads, block_size, head_dim) || num_seqs < 0 ||
      num_tokens < 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      max_query_len < 0 || max_seq_len < 0 || max_query_len > max_seq_len ||
      !valid_scale(k_scale) || !valid_scale(v_scale))
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
  const float scale_log2 = scale * kLog2e * k_scale;
  // One split covering the whole key range: no partials, no workspace.
  const int32_t pps = static_cast<int32_t>(ceil_div(max_seq_len > 0 ? max_seq_len : 1, block_size));
  const int32_t key_cap = std::min(block_table_stride, pps) * block_size;
  const int64_t scratch_blocks = static_cast<int64_t>(num_seqs) * block_table_stride;
  // The MFMA kernel takes row maxima of raw scores, which needs a positive scale.
  const bool mfma_shape =
      scale_log2 > 0.f && scale_log2 < INFINITY &&
      prefill_mfma_supported(dtype, head_dim, G, key_cap, block_size,
                             fp8_pools ? scratch_blocks : num_blocks, num_kv_heads) &&
      aligned16(query) && aligned16(key_cache) && aligned16(value_cache) &&
      q_token_stride % 8 == 0 && q_head_stride % 8 == 0;
  if (mfma_shape && !fp8_pools) {
    PrefillArgs p{query,    q_token_stride, q_head_stride, key_cache,    value_cache,
                  pool,     block_tables,   block_table_stride, seq_lens, cu_seqlens_q,
                  scale_log2, key_cap,      out,           out_token_stride, out_head_stride};
    p.seq_order = seq_order;
    p.num_seqs = num_seqs;
    return launch_prefill_mfma(p, dtype, num_seqs, num_kv_heads, G, head_dim, max_query_len, s);
  }
  if (mfma_shape) {
    // fp8 pools: decode the batch's pages into the scratch pool, then the MFMA
    // kernel reads it through the identity table.
    const ScratchPages sp =
        carve_pages(workspace, num_seqs, block_table_stride, num_kv_heads, block_size, head_dim);
    if (workspace == nullptr || workspace_bytes < sp.bytes || !aligned16(workspace))
      return TKS_ERR_WORKSPACE;
    const int64_t items = scratch_blocks * num_kv_heads * block_size * head_dim / 16;
    const dim3 grid(static_cast<unsigned>(ceil_div(items, 256)));
    const fp8e4m3_t *k8 = static_cast<const fp8e4m3_t *>(key_cache);
    const fp8e4m3_t *v8 = static_cast<const fp8e4m3_t *>(value_cache);
    if (dtype == TKS_BFLOAT16)
      decode_pages_kernel<bf16_t><<<grid, 256, 0, s>>>(
          k8, v8, pool, num_kv_heads, block_tables, block_table_stride, seq_lens, num_seqs,
          static_cast<bf16_t *>(sp.k), static_cast<bf16_t *>(sp.v), sp.table, k_rs, v_rs);
    else
      decode_pages_kernel<_Float16><<<grid, 256, 0, s>>>(
          k8, v8, pool, num_kv_heads, block_tables, block_table_stride, seq_lens, num_seqs,
          static_cast<_Float16 *>(sp.k), static_cast<_Float16 *>(sp.v), sp.table, k_rs, v_rs);
    const int32_t st = check_launch();
    if (st != TKS_OK) return st;
    const PoolView scratch = make_pool(0, scratch_blocks, num_kv_heads, block_size, head_dim);
    PrefillArgs p{query,    q_token_stride, q_head_stride, sp.k,        sp.v,
                  scratch,  sp.table,       block_table_stride, seq_lens, cu_seqlens_q,
                  scale_log2, key_cap,      out,           out_token_stride, out_head_stride};
    p.v_scale = v_scale;
    p.seq_order = seq_order;
    p.num_seqs = num_seqs;
    return launch_prefill_mfma(p, dtype, num_seqs, num_kv_heads, G, head_dim, max_query_len, s);
  }
  const int kv_elem = fp8_pools ? 1 : elem_bytes(dtype);
  GenericArgs a{query,     q_token_stride, q_head_stride, key_cache,  value_cache, pool,
                block_tables, block_table_stride, seq_lens, nullptr, cu_seqlens_q, num_seqs, num_q_heads,
                G,         scale_log2,     pps,           1,          key_cap,     out,         out_token_stride,
                out_head_stride, nullptr,  nullptr,       nullptr,
                vec_rows_ok(key_cache, value_cache, head_dim, kv_elem), v_scale};
  a.k_rs = k_rs;
  a.v_rs = v_rs;
  return launch_generic(a, dtype, static_cast<int32_t>(num_tokens), num_kv_heads, fp8_pools, s);
}

// Device address of `scratch` on the calling thread's current device, looked
// up once per device (with that device current) and kept.
constexpr int kMaxScratchDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mutex;

int32_t scratch_address(void **ptr) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) {
    set_hip_error(err);
    return TKS_ERR_LAUNCH;
  }
  if (device < 0 || device >= kMaxScratchDevices) return TKS_ERR_VALUE;
  void *known = g_scratch_ptr[device].load(std::memory_order_acquire);
  if (known == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    known = g_scratch_ptr[device].load(std::memory_order_relaxed);
    if (known == nullptr) {
      err = hipGetSymbolAddress(&known, HIP_SYMBOL(scratch));
      if (err != hipSuccess || known == nullptr) {
        set_hip_error(err != hipSuccess ? err : hipErrorInvalidSymbol);
        return TKS_ERR_LAUNCH;
      }
      g_scratch_ptr[device].store(known, std::memory_order_release);
    }
  }
  *ptr = known;
  return TKS_OK;
}

}  // namespace

extern "C" int64_t tks_paged_attention_decode_noalloc_max_workspace_bytes(void) {
  return kStaticScratchBytes;
}

extern "C" int32_t tks_paged_attention_decode_noalloc(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *seq_order,
    int32_t num_seqs, int32_t num_q_heads, int32_t max_seq_len, float scale,
    int32_t pages_per_split, void *out, int64_t out_seq_stride, int64_t out_head_stride,
    int32_t dtype, tks_stream_t stream) {
  const int64_t needed = tks_paged_attention_decode_workspace_bytes(
      num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, pages_per_split);
  if (needed < 0) return TKS_ERR_VALUE;
  if (needed > kStaticScratchBytes) return TKS_ERR_WORKSPACE;
  void *ws = nullptr;
  if (needed > 0) {
    const int32_t st = scratch_address(&ws);
    if (st != TKS_OK) return st;
  }
  return decode_impl(query, q_seq_stride, q_head_stride, key_cache, value_cache, num_layers,
                     num_blocks, num_kv_heads, block_size, head_dim, layer_index, block_tables,
                     block_table_stride, seq_lens, seq_order, num_seqs, num_q_heads, max_seq_len,
                     scale, pages_per_split, out, out_seq_stride, out_head_stride, ws,
                     needed > 0 ? kStaticScratchBytes : 0, false, 1.f, 1.f, dtype, stream);
}

extern "C" int32_t tks_paged_attention_decode(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *seq_order, int32_t num_seqs,
    int32_t num_q_heads,
    int32_t max_seq_len, float scale, int32_t pages_per_split, void *out,
    int64_t out_seq_stride, int64_t out_head_stride, void *workspace, int64_t workspace_bytes,
    int32_t dtype, tks_stream_t stream) {
  return decode_impl(query, q_seq_stride, q_head_stride, key_cache, value_cache, num_layers,
                     num_blocks, num_kv_heads, block_size, head_dim, layer_index, block_tables,
                     block_table_stride, seq_lens, seq_order, num_seqs, num_q_heads, max_seq_len,
                     scale, pages_per_split, out, out_seq_stride, out_head_stride, workspace,
                     workspace_bytes, false, 1.f, 1.f, dtype, stream);
}

namespace {

int32_t rope_append_decode_entry(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key,
    int64_t k_seq_stride, int64_t k_head_stride, const void *value, int64_t v_seq_stride,
    int64_t v_head_stride, const int64_t *positions, const void *cos_cache,
    const void *sin_cache, int64_t cache_len, const int64_t *slot_mapping, void *key_cache,
    void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *seq_order,
    int32_t num_seqs, int32_t num_q_heads, int32_t max_seq_len, float scale,
    int32_t pages_per_split, void *out, int64_t out_seq_stride, int64_t out_head_stride,
    void *workspace, int64_t workspace_bytes, bool fp8_pools, float k_scale, float v_scale,
    int32_t dtype, tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (head_dim < 2 || head_dim % 2 != 0 || cache_len <= 0 || num_seqs < 0) return TKS_ERR_VALUE;
  if (num_seqs > 0 && (!key || !value || !positions || !cos_cache || !sin_cache || !slot_mapping))
    return TKS_ERR_VALUE;
  const RopeAppend ra{key,       k_seq_stride, k_head_stride, value,     v_seq_stride,
                      v_head_stride, positions, cos_cache,  sin_cache, cache_len,
                      slot_mapping};
  return decode_impl(query, q_seq_stride, q_head_stride, key_cache, value_cache, num_layers,
                     num_blocks, num_kv_heads, block_size, head_dim, layer_index, block_tables,
                     block_table_stride, seq_lens, seq_order, num_seqs, num_q_heads, max_seq_len,
                     scale, pages_per_split, out, out_seq_stride, out_head_stride, workspace,
                     workspace_bytes, fp8_pools, k_scale, v_scale, dtype, stream, &ra);
}

}  // namespace

extern "C" int32_t tks_rope_append_paged_decode(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key,
    int64_t k_seq_stride, int64_t k_head_stride, const void *value, int64_t v_seq_stride,
    int64_t v_head_stride, const int64_t *positions, const void *cos_cache,
    const void *sin_cache, int64_t cache_len, const int64_t *slot_mapping, void *key_cache,
    void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *seq_order,
    int32_t num_seqs, int32_t num_q_heads, int32_t max_seq_len, float scale,
    int32_t pages_per_split, void *out, int64_t out_seq_stride, int64_t out_head_stride,
    void *workspace, int64_t workspace_bytes, int32_t dtype, tks_stream_t stream) {
  return rope_append_decode_entry(
      query, q_seq_stride, q_head_stride, key, k_seq_stride, k_head_stride, value, v_seq_stride,
      v_head_stride, positions, cos_cache, sin_cache, cache_len, slot_mapping, key_cache,
      value_cache, num_layers, num_blocks, num_kv_heads, block_size, head_dim, layer_index,
      block_tables, block_table_stride, seq_lens, seq_order, num_seqs, num_q_heads, max_seq_len,
      scale, pages_per_split, out, out_seq_stride, out_head_stride, workspace, workspace_bytes,
      false, 1.f, 1.f, dtype, stream);
}

extern "C" int32_t tks_rope_append_paged_decode_fp8(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key,
    int64_t k_seq_stride, int64_t k_head_stride, const void *value, int64_t v_seq_stride,
    int64_t v_head_stride, const int64_t *positions, const void *cos_cache,
    const void *sin_cache, int64_t cache_len, const int64_t *slot_mapping, void *key_cache,
    void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *seq_order,
    int32_t num_seqs, int32_t num_q_heads, int32_t max_seq_len, float scale,
    int32_t pages_per_split, void *out, int64_t out_seq_stride, int64_t out_head_stride,
    void *workspace, int64_t workspace_bytes, float k_scale, float v_scale, int32_t dtype,
    tks_stream_t stream) {
  return rope_append_decode_entry(
      query, q_seq_stride, q_head_stride, key, k_seq_stride, k_head_stride, value, v_seq_stride,
      v_head_stride, positions, cos_cache, sin_cache, cache_len, slot_mapping, key_cache,
      value_cache, num_layers, num_blocks, num_kv_heads, block_size, head_dim, layer_index,
      block_tables, block_table_stride, seq_lens, seq_order, num_seqs, num_q_heads, max_seq_len,
      scale, pages_per_split, out, out_seq_stride, out_head_stride, workspace, workspace_bytes,
      true, k_scale, v_scale, dtype, stream);
}

extern "C" int32_t tks_paged_attention_decode_fp8(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *seq_order,
    int32_t num_seqs, int32_t num_q_heads, int32_t max_seq_len, float scale,
    int32_t pages_per_split, void *out, int64_t out_seq_stride, int64_t out_head_stride,
    void *workspace, int64_t workspace_bytes, float k_scale, float v_scale, int32_t dtype,
    tks_stream_t stream) {
  return decode_impl(query, q_seq_stride, q_head_stride, key_cache, value_cache, num_layers,
                     num_blocks, num_kv_heads, block_size, head_dim, layer_index, block_tables,
                     block_table_stride, seq_lens, seq_order, num_seqs, num_q_heads, max_seq_len,
                     scale, pages_per_split, out, out_seq_stride, out_head_stride, workspace,
                     workspace_bytes, true, k_scale, v_scale, dtype, stream);
}

extern "C" int32_t tks_paged_attention_prefill(
    const void *query, int64_t q_token_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *cu_seqlens_q,
    const int32_t *seq_order, int32_t num_seqs, int64_t num_tokens, int32_t num_q_heads,
    int32_t max_query_len, int32_t max_seq_len, float scale, void *out, int64_t out_token_stride,
    int64_t out_head_stride, int32_t dtype, tks_stream_t stream) {
  return prefill_impl(query, q_token_stride, q_head_stride, key_cache, value_cache, num_layers,
                      num_blocks, num_kv_heads, block_size, head_dim, layer_index, block_tables,
                      block_table_stride, seq_lens, cu_seqlens_q, seq_order, num_seqs, num_tokens,
                      num_q_heads, max_query_len, max_seq_len, scale, out, out_token_stride,
                      out_head_stride, false, nullptr, 0, 1.f, 1.f, dtype, stream);
}

extern "C" int64_t tks_paged_attention_prefill_fp8_workspace_bytes(
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t block_table_stride, int32_t max_seq_len, int32_t dtype) {
  if (num_seqs < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      block_size <= 0 || block_table_stride < 0 || max_seq_len < 0 ||
      num_q_heads % num_kv_heads != 0 || !valid_dtype(dtype))
    return -1;
  const int32_t pps = static_cast<int32_t>(ceil_div(max_seq_len > 0 ? max_seq_len : 1, block_size));
  const int32_t key_cap = std::min(block_table_stride, pps) * block_size;
  const int64_t scratch_blocks = static_cast<int64_t>(num_seqs) * block_table_stride;
  if (!prefill_mfma_supported(dtype, head_dim, num_q_heads / num_kv_heads, key_cap, block_size,
                              scratch_blocks, num_kv_heads))
    return 0;
  return carve_pages(nullptr, num_seqs, block_table_stride, num_kv_heads, block_size, head_dim)
      .bytes;
}

extern "C" int32_t tks_paged_attention_prefill_fp8(
    const void *query, int64_t q_token_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *cu_seqlens_q,
    const int32_t *seq_order, int32_t num_seqs, int64_t num_tokens, int32_t num_q_heads,
    int32_t max_query_len, int32_t max_seq_len, float scale, void *out, int64_t out_token_stride,
    int64_t out_head_stride, void *workspace, int64_t workspace_bytes, float k_scale,
    float v_scale, int32_t dtype, tks_stream_t stream) {
  return prefill_impl(query, q_token_stride, q_head_stride, key_cache, value_cache, num_layers,
                      num_blocks, num_kv_heads, block_size, head_dim, layer_index, block_tables,
                      block_table_stride, seq_lens, cu_seqlens_q, seq_order, num_seqs, num_tokens,
                      num_q_heads, max_query_len, max_seq_len, scale, out, out_token_stride,
                      out_head_stride, true, workspace, workspace_bytes, k_scale, v_scale, dtype,
                      stream);
}

// ------------------------------------------------------------------------
// fp8 pools with one scale per pool row: the per-pool entries with the scale
// arrays in place of the two scales (which are then 1).
// ------------------------------------------------------------------------

extern "C" int32_t tks_paged_attention_decode_fp8_rows(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, const float *k_scales, const float *v_scales, int32_t num_layers,
    int64_t num_blocks, int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
    int32_t layer_index, const int32_t *block_tables, int32_t block_table_stride,
    const int32_t *seq_lens, const int32_t *seq_order, int32_t num_seqs, int32_t num_q_heads,
    int32_t max_seq_len, float scale, int32_t pages_per_split, void *out,
    int64_t out_seq_stride, int64_t out_head_stride, void *workspace, int64_t workspace_bytes,
    int32_t dtype, tks_stream_t stream) {
  if (num_seqs > 0 && (!k_scales || !v_scales)) return TKS_ERR_VALUE;
  return decode_impl(query, q_seq_stride, q_head_stride, key_cache, value_cache, num_layers,
                     num_blocks, num_kv_heads, block_size, head_dim, layer_index, block_tables,
                     block_table_stride, seq_lens, seq_order, num_seqs, num_q_heads, max_seq_len,
                     scale, pages_per_split, out, out_seq_stride, out_head_stride, workspace,
                     workspace_bytes, true, 1.f, 1.f, dtype, stream, nullptr, k_scales,
                     v_scales);
}

extern "C" int32_t tks_paged_attention_prefill_fp8_rows(
    const void *query, int64_t q_token_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, const float *k_scales, const float *v_scales, int32_t num_layers,
    int64_t num_blocks, int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
    int32_t layer_index, const int32_t *block_tables, int32_t block_table_stride,
    const int32_t *seq_lens, const int32_t *cu_seqlens_q, const int32_t *seq_order,
    int32_t num_seqs, int64_t num_tokens, int32_t num_q_heads, int32_t max_query_len,
    int32_t max_seq_len, float scale, void *out, int64_t out_token_stride,
    int64_t out_head_stride, void *workspace, int64_t workspace_bytes, int32_t dtype,
    tks_stream_t stream) {
  if (num_seqs > 0 && num_tokens > 0 && (!k_scales || !v_scales)) return TKS_ERR_VALUE;
  return prefill_impl(query, q_token_stride, q_head_stride, key_cache, value_cache, num_layers,
                      num_blocks, num_kv_heads, block_size, head_dim, layer_index, block_tables,
                      block_table_stride, seq_lens, cu_seqlens_q, seq_order, num_seqs, num_tokens,
                      num_q_heads, max_query_len, max_seq_len, scale, out, out_token_stride,
                      out_head_stride, true, workspace, workspace_bytes, 1.f, 1.f, dtype, stream,
                      k_scales, v_scales);
}

extern "C" int32_t tks_rope_append_paged_decode_fp8_rows(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key,
    int64_t k_seq_stride, int64_t k_head_stride, const void *value, int64_t v_seq_stride,
    int64_t v_head_stride, const int64_t *positions, const void *cos_cache,
    const void *sin_cache, int64_t cache_len, const int64_t *slot_mapping, void *key_cache,
    void *value_cache, float *k_scales, float *v_scales, int32_t num_layers,
    int64_t num_blocks, int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
    int32_t layer_index, const int32_t *block_tables, int32_t block_table_stride,
    const int32_t *seq_lens, const int32_t *seq_order, int32_t num_seqs, int32_t num_q_heads,
    int32_t max_seq_len, float scale, int32_t pages_per_split, void *out,
    int64_t out_seq_stride, int64_t out_head_stride, void *workspace, int64_t workspace_bytes,
    int32_t dtype, tks_stream_t stream) {
  if (!valid_dtype(dtype)) return TKS_ERR_TYPE;
  if (head_dim < 2 || head_dim % 2 != 0 || cache_len <= 0 || num_seqs < 0) return TKS_ERR_VALUE;
  if (num_seqs > 0 && (!key || !value || !positions || !cos_cache || !sin_cache ||
                       !slot_mapping || !k_scales || !v_scales))
    return TKS_ERR_VALUE;
  const RopeAppend ra{key,       k_seq_stride, k_head_stride, value,     v_seq_stride,
                      v_head_stride, positions, cos_cache,  sin_cache, cache_len,
                      slot_mapping};
  return decode_impl(query, q_seq_stride, q_head_stride, key_cache, value_cache, num_layers,
                     num_blocks, num_kv_heads, block_size, head_dim, layer_index, block_tables,
                     block_table_stride, seq_lens, seq_order, num_seqs, num_q_heads, max_seq_len,
                     scale, pages_per_split, out, out_seq_stride, out_head_stride, workspace,
                     workspace_bytes, true, 1.f, 1.f, dtype, stream, &ra, k_scales, v_scales);
}
