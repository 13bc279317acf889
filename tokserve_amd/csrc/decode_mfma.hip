// Paged decode with MFMA scores, bf16/fp16, block size 16.
//
// Two kernels. decode_pv_kernel (further below) is the one every launch takes: both
// products on the MFMA pipe, K/V pages HBM -> LDS by DMA. decode_mfma_kernel, the
// earlier design described next, computes P.V on the VALU; it is compiled only with
// kPvMfma set to false, to compare the two.
//
// decode_mfma_kernel: one workgroup of NW waves per (sequence, KV head[, split]). The pages of the
// sequence are cut into NW contiguous ranges, one per wave; the waves' partial
// softmax states (m, l, acc) are merged through LDS at the end, so no result
// ever crosses workgroups inside the kernel (a cross-workgroup split, used only
// for batches too small to fill the GPU, is merged by a second launch).
//
// Per page (16 x Dh contiguous elements of one KV head = one MFMA tile):
//   S^T (16 rows x 16 tokens) = Q_rep . K^T   with v_mfma_f32_16x16x32_{bf16,f16}
//     A operand: row m holds query head m % G of this KV group (replicated),
//     B operand: column n holds token n of the page, straight from 16-byte
//     HBM loads (lane (grp, r) reads dims c*32 + grp*8 .. +8 of token r);
//     lane (grp, r) receives the scores of heads (grp*4 + i) % G for token r.
// Softmax is online with a lazy reference: each lane checks its own scores
// against reference + 8 (log2 units), and only when some score passes it does
// the wave take row maxima, move the reference and rescale l and the P.V
// accumulators (rare after a row's first page). The page's probabilities
// (G x 16) go through a per-wave LDS slice. P.V runs on the VALU as packed
// two-element dot products (v_dot2_f32_bf16 / _f16: P rounded to the model
// dtype, V exact, fp32 accumulation): lane (hg, tg, dc) owns dims dc*8 .. +8
// of heads hg*HPL .. +HPL and tokens tg*4 .. +3 of every page, so V also
// arrives as 16-byte (fp8: 8-byte) loads, regrouped into token pairs by byte
// permutes; the four token groups are summed once per wave. Every K/V byte is read from HBM exactly once
// for all G query heads. Pages are double-buffered in registers and a wave's
// block ids sit in one VGPR (broadcast with readlane), so nothing in the page
// loop waits on a dependent memory access.
#include "attention_common.hpp"
#include "rope_common.hpp"

namespace tks {
namespace {

constexpr int kWaves = 4;
// s_waitcnt immediate: vmcnt 0, expcnt and lgkmcnt left at their maxima (no wait).
constexpr int kWaitVmcntZero = 0x0F70;
// Register pages per wave: the page being consumed and the next one in flight
// (3 or 4 measured no faster, for bf16 and for fp8 pages, and cost occupancy).
// (3 or 4 pages measured no faster at Dh 64 either, also at batches of two waves
// per SIMD: there the page loop is bound by its own instruction latency.)
constexpr int kRing = 2;

template <int DH, int G>
struct DecodeShape {
  static constexpr int BS = 16;
  static constexpr int NC = DH / 32;                // QK k-chunks of 32
  static constexpr int LPR = DH / 8;                // lanes per V row (8 dims each)
  static constexpr int TG = 4;                      // token groups (4 tokens each)
  static constexpr int HG = 64 / (LPR * TG);        // head groups across the wave
  static constexpr int HPL = G / HG;                // heads per lane in P.V
  static_assert(DH == 64 || DH == 128, "head_dim");
  static_assert(HG >= 1 && G % HG == 0 && 16 % G == 0, "group size");
  static_assert(HPL * 8 <= 64, "P.V accumulator budget");
};

// Orders LDS traffic among the lanes of one wave (the waves of a workgroup run
// different page counts, so a workgroup barrier cannot be used in the loop).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Packed pairs of the model dtype for the P.V dot products.
template <typename T>
struct Dot2;
template <>
struct Dot2<bf16_t> {
  typedef __bf16 pair __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float run(pair a, pair b, float c) {
#if __HIP_DEVICE_COMPILE__
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
#else
    return c;
#endif
  }
  // Two e4m3 codes of a word (bytes 0, 1, or 2, 3 with HI) as a pair, exactly.
  template <bool HI>
  static __device__ __forceinline__ pair from_fp8(uint32_t w) {
#if __HIP_DEVICE_COMPILE__
    return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI);
#else
    (void)w;
    return pair{};
#endif
  }
};
template <>
struct Dot2<_Float16> {
  typedef _Float16 pair __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float run(pair a, pair b, float c) {
#if __HIP_DEVICE_COMPILE__
    return __builtin_amdgcn_fdot2(a, b, c, false);
#else
    return c;
#endif
  }
  template <bool HI>
  static __device__ __forceinline__ pair from_fp8(uint32_t w) {
#if __HIP_DEVICE_COMPILE__
    return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI);
#else
    (void)w;
    return pair{};
#endif
  }
};

template <typename P>
__device__ __forceinline__ P pair_bits(uint32_t w) {
  P r;
  __builtin_memcpy(&r, &w, 4);
  return r;
}

// Byte permute: byte i of the result is byte sel_i of (hi : lo), bytes 0-3 from
// lo and 4-7 from hi.
__device__ __forceinline__ uint32_t byte_perm(uint32_t hi, uint32_t lo, uint32_t sel) {
#if __HIP_DEVICE_COMPILE__
  return __builtin_amdgcn_perm(hi, lo, sel);
#else
  (void)hi, (void)sel;
  return lo;
#endif
}

// K/V rows as stored: T itself, or fp8 e4m3 decoded exactly to T (every e4m3
// value is a bf16 and an f16), K as MFMA operands and V as token pairs for the
// dot products. A lane's 8 elements of a row are one 16-byte load of T or one
// 8-byte load of fp8.
template <typename T, typename KV>
struct PageIO {
  typedef uint4 raw;
  typedef typename Dot2<T>::pair pair;
  static __device__ __forceinline__ raw load(const KV *p) { return ld16_stream(p); }
  static __device__ __forceinline__ typename Mfma<T>::v8 k_operand(raw r) { return as_v8<T>(r); }
  // Rows t0, t1 (8 elements each) as token pairs: vp[d] = {row t0[d], row t1[d]}.
  static __device__ __forceinline__ void v_pairs(raw t0, raw t1, pair (&vp)[8]) {
    const uint32_t a[4] = {t0.x, t0.y, t0.z, t0.w}, b[4] = {t1.x, t1.y, t1.z, t1.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      vp[2 * k] = pair_bits<pair>(byte_perm(b[k], a[k], 0x05040100u));
      vp[2 * k + 1] = pair_bits<pair>(byte_perm(b[k], a[k], 0x07060302u));
    }
  }
  static __device__ __forceinline__ raw zero() { return make_uint4(0, 0, 0, 0); }
};
template <typename T>
struct PageIO<T, fp8e4m3_t> {
  typedef uint2 raw;
  static __device__ __forceinline__ raw load(const fp8e4m3_t *p) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
    return make_uint2(v.x, v.y);
  }
  static __device__ __forceinline__ typename Mfma<T>::v8 k_operand(raw r) {
    typename Mfma<T>::v8 o = {};
#if __HIP_DEVICE_COMPILE__
    const uint32_t w[2] = {r.x, r.y};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if constexpr (__is_same(T, bf16_t)) {
        const auto lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[i], 1.0f, false);
        const auto hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[i], 1.0f, true);
        o[4 * i] = lo[0];
        o[4 * i + 1] = lo[1];
        o[4 * i + 2] = hi[0];
        o[4 * i + 3] = hi[1];
      } else {
        const auto lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[i], 1.0f, false);
        const auto hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[i], 1.0f, true);
        o[4 * i] = lo[0];
        o[4 * i + 1] = lo[1];
        o[4 * i + 2] = hi[0];
        o[4 * i + 3] = hi[1];
      }
    }
#else
    (void)r;
#endif
    return o;
  }
  typedef typename Dot2<T>::pair pair;
  // Rows t0, t1 (8 e4m3 codes each) as token pairs of T, decoded exactly: the
  // permutes put (t0[d], t1[d]) side by side, one conversion decodes a pair.
  static __device__ __forceinline__ void v_pairs(raw t0, raw t1, pair (&vp)[8]) {
    const uint32_t a[2] = {t0.x, t0.y}, b[2] = {t1.x, t1.y};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t x = byte_perm(b[k], a[k], 0x05010400u);  // t0.0 t1.0 t0.1 t1.1
      const uint32_t y = byte_perm(b[k], a[k], 0x07030602u);  // t0.2 t1.2 t0.3 t1.3
      vp[4 * k] = Dot2<T>::template from_fp8<false>(x);
      vp[4 * k + 1] = Dot2<T>::template from_fp8<true>(x);
      vp[4 * k + 2] = Dot2<T>::template from_fp8<false>(y);
      vp[4 * k + 3] = Dot2<T>::template from_fp8<true>(y);
    }
  }
  static __device__ __forceinline__ raw zero() { return make_uint2(0, 0); }
};

template <bool B>
struct BoolConst {
  static constexpr bool value = B;
};

// Eight values of a row chunk, held at T's precision, as the pool stores them: T
// elements (16 bytes) or e4m3 codes of value / scale (8 bytes).
template <typename T, typename KV>
__device__ __forceinline__ typename PageIO<T, KV>::raw pool_chunk(const float *x, float scale) {
  if constexpr (sizeof(KV) == 1) {
    uint32_t w[2];
    e4m3_words<8>(x, scale, w);
    return make_uint2(w[0], w[1]);
  } else {
    (void)scale;
    return pack<T>(x);
  }
}

template <typename T, typename KV>
__device__ __forceinline__ void store_chunk(KV *dst, typename PageIO<T, KV>::raw v) {
  if constexpr (sizeof(KV) == 1)
    *reinterpret_cast<uint2 *>(dst) = v;
  else
    st16(dst, v);
}

// The fused append, in two steps run by one wave per (sequence, KV head). First
// the new rows are staged in LDS (k_s, v_s: Dh entries each, in the pool's form):
// sequence b's key row rotated at its position and its value row, as T or, over
// e4m3 pools, as the codes of the rotated row (rounded to T first) and of the value
// row; lanes t < 3 Dh / 16 take part (every lane of the wave with ROWS, where each
// row has a scale of its own). Returns whether slot a.slots[b] lies in the pool (a
// negative slot appends nothing).
template <typename T, typename KV, int DH, int BS, bool ROWS = false>
__device__ __forceinline__ bool stage_new_rows(const DecodeArgs &a, int b, int kvh, int t,
                                               KV *k_s, KV *v_s, float *scale_s = nullptr) {
  constexpr int HALF = DH / 2;
  const int64_t slot = a.slots[b];
  if (slot < 0 || slot >= a.pool.num_blocks * BS) return false;
  if constexpr (ROWS) {
    // One scale per row (amax / 448 over its Dh values, the key's after the
    // rotation and its rounding to T): wave maxima over the lanes holding each row,
    // so every lane of the wave takes part; the scales go to scale_s[0..1].
    static_assert(sizeof(KV) == 1, "row scales: fp8 pools");
    const bool kl = t < HALF / 8;
    const bool vl = !kl && t < HALF / 8 + DH / 8;
    float o1[8], o2[8], x[8];
    float kmax = 0.f, vmax = 0.f;
    if (kl) {
      const T *kn = static_cast<const T *>(a.k_new) + b * a.kn_ss + (int64_t)kvh * a.kn_hs;
      const int64_t pos = min(max(a.positions[b], (int64_t)0), a.table_len - 1);
      float cf[8], sf[8];
      load_table<T, 8>(static_cast<const T *>(a.cos_t) + pos * HALF,
                       static_cast<const T *>(a.sin_t) + pos * HALF, t * 8, cf, sf);
      rotate_values<T, 8>(kn + t * 8, cf, sf, HALF, o1, o2);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o1[e] = round_through<T>(o1[e]);
        o2[e] = round_through<T>(o2[e]);
        kmax = abs_max_nan(abs_max_nan(kmax, o1[e]), o2[e]);
      }
    } else if (vl) {
      const T *vn = static_cast<const T *>(a.v_new) + b * a.vn_ss + (int64_t)kvh * a.vn_hs;
      unpack<T>(ld16(vn + (t - HALF / 8) * 8), x);
#pragma unroll
      for (int e = 0; e < 8; ++e) vmax = abs_max_nan(vmax, x[e]);
    }
    const float ks = row_scale_of(wave_abs_max(kmax));
    const float vs = row_scale_of(wave_abs_max(vmax));
    if (kl) {
      store_chunk<T, KV>(k_s + t * 8, pool_chunk<T, KV>(o1, ks));
      store_chunk<T, KV>(k_s + t * 8 + HALF, pool_chunk<T, KV>(o2, ks));
    } else if (vl) {
      store_chunk<T, KV>(v_s + (t - HALF / 8) * 8, pool_chunk<T, KV>(x, vs));
    }
    if (t == 0) {
      scale_s[0] = ks;
      scale_s[1] = vs;
    }
    return true;
  }
  if (t < HALF / 8) {
    const T *kn = static_cast<const T *>(a.k_new) + b * a.kn_ss + (int64_t)kvh * a.kn_hs;
    const int64_t pos = min(max(a.positions[b], (int64_t)0), a.table_len - 1);
    float cf[8], sf[8], o1[8], o2[8];
    load_table<T, 8>(static_cast<const T *>(a.cos_t) + pos * HALF,
                     static_cast<const T *>(a.sin_t) + pos * HALF, t * 8, cf, sf);
    rotate_values<T, 8>(kn + t * 8, cf, sf, HALF, o1, o2);
    if constexpr (sizeof(KV) == 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o1[e] = round_through<T>(o1[e]);
        o2[e] = round_through<T>(o2[e]);
      }
      store_chunk<T, KV>(k_s + t * 8, pool_chunk<T, KV>(o1, a.k_scale));
      store_chunk<T, KV>(k_s + t * 8 + HALF, pool_chunk<T, KV>(o2, a.k_scale));
    } else {
      store_chunk<T, KV>(k_s + t * 8, pack<T>(o1));
      store_chunk<T, KV>(k_s + t * 8 + HALF, pack<T>(o2));
    }
  } else if (t < HALF / 8 + DH / 8) {
    const T *vn = static_cast<const T *>(a.v_new) + b * a.vn_ss + (int64_t)kvh * a.vn_hs;
    const int c = (t - HALF / 8) * 8;
    if constexpr (sizeof(KV) == 1) {
      float x[8];
      unpack<T>(ld16(vn + c), x);
      store_chunk<T, KV>(v_s + c, pool_chunk<T, KV>(x, a.v_scale));
    } else {
      store_chunk<T, KV>(v_s + c, ld16(vn + c));
    }
  }
  return true;
}

// Eight pool elements at p (LDS) in the kernel's page-register form.
template <typename T, typename KV>
__device__ __forceinline__ typename PageIO<T, KV>::raw load_chunk(const KV *p) {
  if constexpr (sizeof(KV) == 1)
    return *reinterpret_cast<const uint2 *>(p);
  else
    return ld16(p);
}

// Then the staged rows go from LDS to pool slot a.slots[b] (lanes t < Dh / 4; the
// slot was checked by stage_new_rows).
// ROWS: lanes 0 and Dh / 8 also store the rows' scales from scale_s to their slot
// of the scale arrays.
template <typename T, typename KV, int DH, int BS, bool ROWS = false>
__device__ __forceinline__ void write_staged_rows(const DecodeArgs &a, int b, int kvh, int t,
                                                  const KV *k_s, const KV *v_s,
                                                  const float *scale_s = nullptr) {
  if (t >= DH / 4) return;
  const int64_t slot = a.slots[b];
  const int64_t blk = slot / BS;
  const int64_t row = a.pool.layer_base + blk * a.pool.block_stride +
                      (int64_t)kvh * a.pool.head_stride + (slot - blk * BS) * DH;
  const bool is_k = t < DH / 8;
  const int c = (is_k ? t : t - DH / 8) * 8;
  KV *dst = static_cast<KV *>(const_cast<void *>(is_k ? a.kc : a.vc)) + row + c;
  store_chunk<T, KV>(dst, load_chunk<T, KV>((is_k ? k_s : v_s) + c));
  if constexpr (ROWS) {
    if (c == 0) const_cast<float *>(is_k ? a.k_rs : a.v_rs)[row / DH] = scale_s[is_k ? 0 : 1];
  }
}

// ROPE: RoPE and the KV append of the sequence's new token fused in (DecodeArgs).
// Every workgroup rotates its query rows as it loads them; the wave that reads the
// sequence's last page stages the rotated key row and the value row in LDS, uses
// them in place of what it loads of their slot and writes them to the pool after
// its page loop, so no workgroup reads pool memory written in the same launch.
// ROWS: fp8 pools with one scale per pool row (a.k_rs, a.v_rs); lane r of a page
// loads its token's two scales with the page, multiplies its scores by the key
// scale and its probabilities (after they enter the row sum) by the value scale.
template <typename T, typename KV, int DH, int G, bool ROPE, bool ROWS = false>
__global__ __launch_bounds__(64 * kWaves) void decode_mfma_kernel(DecodeArgs a) {
  using S = DecodeShape<DH, G>;
  constexpr int BS = S::BS, NC = S::NC, LPR = S::LPR, TG = S::TG, HPL = S::HPL;
  using M = Mfma<T>;
  using IO = PageIO<T, KV>;
  using raw = typename IO::raw;
  __shared__ __attribute__((aligned(16))) float p_s[kWaves][16][BS];  // rows >= G: padding
  __shared__ __attribute__((aligned(16))) float alpha_s[kWaves][G];
  __shared__ __attribute__((aligned(16))) float m_s[kWaves][G];
  __shared__ __attribute__((aligned(16))) float l_s[kWaves][G];
  __shared__ __attribute__((aligned(16))) float acc_s[kWaves][G][DH];
  // The fused append's new key and value rows, in the pool's form, and the
  // workgroup's G query rows (rotated when the RoPE is fused in).
  __shared__ __attribute__((aligned(16))) KV new_k_s[ROPE ? DH : 1];
  __shared__ __attribute__((aligned(16))) KV new_v_s[ROPE ? DH : 1];
  __shared__ __attribute__((aligned(16))) T q_s[G * DH];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;   // QK: token of the page
  const int grp = lane >> 4; // QK: k-group / output row block
  const int dc = lane % LPR;          // P.V: 8-dim chunk
  const int tg = (lane / LPR) % TG;   // P.V: token group
  const int hg = lane / (LPR * TG);   // P.V: head group

  const int kvh = blockIdx.x;
  const int split = blockIdx.z;
  const int b = a.seq_order ? min(max(a.seq_order[blockIdx.y], 0), (int)gridDim.y - 1)
                            : (int)blockIdx.y;
  // A length above the host bound is clamped so no access can leave its buffer.
  const int len = min(a.seq_lens[b], a.key_cap);
  const int n_pages = (len + BS - 1) / BS;
  const int p_begin = split * a.pages_per_split;
  T *out = static_cast<T *>(a.out);
  if (p_begin >= n_pages) {
    if (split == 0) {  // empty sequence: defined all-zero output
      for (int i = threadIdx.x; i < G * DH; i += 64 * kWaves)
        out[b * a.o_ss + (int64_t)(kvh * G + i / DH) * a.o_hs + i % DH] = from_float<T>(0.f);
      if constexpr (ROPE) {
        if (n_pages == 0 && threadIdx.x < 64 &&
            stage_new_rows<T, KV, DH, BS>(a, b, kvh, threadIdx.x, new_k_s, new_v_s)) {
          wave_lds_sync();
          write_staged_rows<T, KV, DH, BS>(a, b, kvh, threadIdx.x, new_k_s, new_v_s);
        }
      }
    }
    return;
  }
  const int p_end = min(n_pages, p_begin + a.pages_per_split);
  const int per_wave = (p_end - p_begin + kWaves - 1) / kWaves;
  const int w_begin = p_begin + wave * per_wave;
  const int w_end = min(p_end, w_begin + per_wave);

  // The QK dot product runs over the dims in any order Q and K share. Pools in
  // the model dtype: MFMA c takes dims c*32 + grp*8 .. +8 (one 16-byte K load
  // each). fp8 pools: lane group grp holds the contiguous slab of dims
  // grp*NC*8 .. +NC*8 and MFMA c its c-th 8 dims, so a lane's K bytes of a page
  // come in NC/2 16-byte loads instead of NC 8-byte ones.
  constexpr bool kSlab = sizeof(KV) == 1;
  typename M::v8 qa[NC];
  // The workgroup's G query rows go through LDS once, a 16-byte chunk per thread
  // (one rotation pair per thread when the RoPE is fused in), and every lane reads
  // its MFMA chunks there: 1-2 % faster than each lane loading its chunks from global
  // memory at small batches, and over e4m3 pools (slab layout, where a rotation
  // pair's halves sit in different lane groups) the way to rotate without cross-lane
  // moves. With the RoPE fused in, the wave whose range holds the sequence's last
  // page stages the new rows in LDS first, so their loads overlap the barrier's wait;
  // its lanes of the new token put them in place of what they load of that page, and
  // after its page loop it writes them to the pool.
  const int32_t *bt_row = a.bt + (int64_t)b * a.bt_stride;
  bool staged = false;  // this wave staged the new rows (it writes them to the pool)
  bool patch = false;   // ... and puts them in place of its loads (length not clamped)
  const int new_off = ROPE ? (len - 1) % BS : 0;
  {
    const int t = threadIdx.x;
    if constexpr (ROPE) {
      constexpr int HALF = DH / 2;
      if (w_begin < w_end && w_end == n_pages) {  // wave-uniform
        staged = stage_new_rows<T, KV, DH, BS>(a, b, kvh, lane, new_k_s, new_v_s);
        patch = staged && a.seq_lens[b] == len;
        wave_lds_sync();
      }
      if (t < G * HALF / 8) {
        const int64_t pos = min(max(a.positions[b], (int64_t)0), a.table_len - 1);
        const int h = t / (HALF / 8), j = (t % (HALF / 8)) * 8;
        const T *qrow =
            static_cast<const T *>(a.q) + b * a.q_ss + (int64_t)(kvh * G + h) * a.q_hs;
        float cf[8], sf[8], o1[8], o2[8];
        load_table<T, 8>(static_cast<const T *>(a.cos_t) + pos * HALF,
                         static_cast<const T *>(a.sin_t) + pos * HALF, j, cf, sf);
        rotate_values<T, 8>(qrow + j, cf, sf, HALF, o1, o2);
        st16(&q_s[h * DH + j], pack<T>(o1));
        st16(&q_s[h * DH + j + HALF], pack<T>(o2));
      }
    } else {
      if (t < G * DH / 8) {
        const int h = t / (DH / 8), j = (t % (DH / 8)) * 8;
        const T *qrow =
            static_cast<const T *>(a.q) + b * a.q_ss + (int64_t)(kvh * G + h) * a.q_hs;
        st16(&q_s[h * DH + j], ld16(qrow + j));
      }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NC; ++c)
      qa[c] = as_v8<T>(ld16(&q_s[(r % G) * DH + (kSlab ? grp * NC * 8 + c * 8 : c * 32 + grp * 8)]));
  }

  const KV *kc = static_cast<const KV *>(a.kc) + a.pool.layer_base + (int64_t)kvh * a.pool.head_stride;
  const KV *vc = static_cast<const KV *>(a.vc) + a.pool.layer_base + (int64_t)kvh * a.pool.head_stride;
  const int k_off = r * DH + grp * (kSlab ? NC * 8 : 8);
  const int v_off = tg * 4 * DH + dc * 8;

  float acc[HPL][8];
#pragma unroll
  for (int j = 0; j < HPL; ++j)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[j][d] = 0.f;
  // Per row i of this lane (head (grp*4 + i) % G, token r): m = reference max
  // in log2 units (-inf before the first key), l = this lane's share of the sum;
  // thr = m + 8 (a score above it moves the reference) and mref = the value
  // subtracted before exp2 (m, or 0 while m is -inf), both updated only when
  // the reference moves.
  float m[4], l[4], thr[4], mref[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
    thr[i] = -INFINITY;
    mref[i] = 0.f;
  }
  const float scale_log2 = a.scale_log2;

  // Row scales of token r of a page: ks_row[blk * rows_per_block].
  const int64_t rows_per_block = a.pool.block_stride / DH;
  const float *ks_row = nullptr;
  const float *vs_row = nullptr;
  if constexpr (ROWS) {
    const int64_t base = (a.pool.layer_base + (int64_t)kvh * a.pool.head_stride) / DH + r;
    ks_row = a.k_rs + base;
    vs_row = a.v_rs + base;
  }
  // Every page is read once: non-temporal loads.
  auto load_page = [&](int blk_reg, int idx, raw (&kr)[NC], raw (&vr)[4], float &ks, float &vs) {
    const int64_t blk = clamp_block(__builtin_amdgcn_readlane(blk_reg, idx), a.pool.num_blocks);
    if constexpr (ROWS) {
      ks = ks_row[blk * rows_per_block];
      vs = vs_row[blk * rows_per_block];
    }
    const KV *kp = kc + blk * a.pool.block_stride + k_off;
    const KV *vp = vc + blk * a.pool.block_stride + v_off;
    if constexpr (kSlab) {
      static_assert(NC % 2 == 0, "fp8 K slab in 16-byte loads");
#pragma unroll
      for (int c = 0; c < NC; c += 2) {
        const uint4 u = ld16_stream(kp + c * 8);
        kr[c] = raw{u.x, u.y};
        kr[c + 1] = raw{u.z, u.w};
      }
    } else {
#pragma unroll
      for (int c = 0; c < NC; ++c) kr[c] = IO::load(kp + c * 32);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) vr[j] = IO::load(vp + j * DH);
  };

  using pair = typename IO::pair;
  // vr is the ring's page: rows past the sequence's last key are zeroed in place
  // (the slot is reloaded before its next use). Only a wave's last page can be
  // the sequence's last page, so the page loop's steady state passes
  // kCheckEnd = false and skips the check; its drain passes true.
  // The fused append's new rows in place of what was loaded of the sequence's last
  // page (only a wave's last page can be it: the page loop's drain).
  auto substitute_new_rows = [&](raw (&kr)[NC], raw (&vr)[4], int p) {
    if (patch && p == n_pages - 1) {
      if (r == new_off) {
#pragma unroll
        for (int c = 0; c < NC; ++c)
          kr[c] = load_chunk<T, KV>(new_k_s + (kSlab ? grp * NC * 8 + c * 8 : c * 32 + grp * 8));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (tg * 4 + j == new_off) vr[j] = load_chunk<T, KV>(new_v_s + dc * 8);
    }
  };
  auto consume = [&](auto check_end, const raw (&kr)[NC], raw (&vr)[4], int p, float ks,
                     float vs) {
    constexpr bool kCheckEnd = decltype(check_end)::value;
    typename M::f4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) s4 = M::run(qa[c], IO::k_operand(kr[c]), s4);
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = s4[i] * scale_log2;
    if constexpr (ROWS) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] *= ks;
    }
    // The sequence's last page (uniform): keys past len score -inf, and their V
    // rows, whatever the pool holds there, are zeroed, since 0 * NaN is NaN.
    if (kCheckEnd && (p + 1) * BS > len) {
      const bool valid = p * BS + r < len;
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] = valid ? sv[i] : -INFINITY;
      if constexpr (ROWS) vs = valid ? vs : 0.f;  // an unwritten row's scale may be NaN
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (p * BS + tg * 4 + j >= len) vr[j] = IO::zero();
    }
    bool over = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) over = over || sv[i] > thr[i];
    // A score more than 8 above its row's reference (every row on the first
    // page): row maxima, new references, l rescaled here and the P.V
    // accumulators below (alpha through LDS).
    const bool rebase = __builtin_amdgcn_ballot_w64(over) != 0;
    if (rebase) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float mx = row16_max(sv[i]);
        const bool bump = mx > thr[i];
        const float alpha = bump ? fast_exp2(m[i] - mx) : 1.f;
        m[i] = bump ? mx : m[i];
        thr[i] = m[i] + 8.f;
        mref[i] = m[i] == -INFINITY ? 0.f : m[i];
        l[i] *= alpha;
        const int h = grp * 4 + i;
        if (h < G && r == 0) alpha_s[wave][h] = alpha;
      }
    }
    // Rows past G (lane groups replicating heads) land in padding rows of p_s.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float pv = fast_exp2(sv[i] - mref[i]);
      l[i] += pv;
      p_s[wave][grp * 4 + i][r] = ROWS ? pv * vs : pv;
    }
    wave_lds_sync();
    pair vp[2][8];
    IO::v_pairs(vr[0], vr[1], vp[0]);
    IO::v_pairs(vr[2], vr[3], vp[1]);
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
      const int h = hg * HPL + j;
      if (rebase) {
        const float al = alpha_s[wave][h];
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[j][d] *= al;
      }
      const float4 pv = *reinterpret_cast<const float4 *>(&p_s[wave][h][tg * 4]);
      pair p01, p23;
      p01[0] = static_cast<typename M::elem>(pv.x);
      p01[1] = static_cast<typename M::elem>(pv.y);
      p23[0] = static_cast<typename M::elem>(pv.z);
      p23[1] = static_cast<typename M::elem>(pv.w);
#pragma unroll
      for (int d = 0; d < 8; ++d)
        acc[j][d] = Dot2<T>::run(vp[1][d], p23, Dot2<T>::run(vp[0][d], p01, acc[j][d]));
    }
    wave_lds_sync();
  };

  // A ring of kRing register pages: the steady-state loop always has the next
  // kRing - 1 pages' loads issued behind the page being consumed (straight-line,
  // so the wait before each consume covers only its own page); the last pages
  // of a 64-page chunk drain in the epilogue.
  constexpr int D = kRing;
  for (int c0 = w_begin; c0 < w_end; c0 += 64) {
    const int n = min(w_end, c0 + 64) - c0;
    const int blk_reg = lane < n ? bt_row[c0 + lane] : 0;
    // Wait for the block ids here, while no page load is in flight (the previous
    // chunk's ring has drained). Without this the compiler, which cannot place this
    // load in the page loop's count of outstanding loads, waits for every load in
    // flight at each loop iteration before it reads a block id, and the register
    // ring never holds more than the one page being consumed.
    __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);
    raw kb[D][NC], vb[D][4];
    float ksr[D] = {}, vsr[D] = {};
#pragma unroll
    for (int j = 0; j < D - 1; ++j)
      if (j < n) load_page(blk_reg, j, kb[j], vb[j], ksr[j], vsr[j]);
    int i = 0;  // page i sits in ring slot i % D
    for (; i + 2 * D - 1 <= n; i += D) {
#pragma unroll
      for (int j = 0; j < D; ++j) {
        load_page(blk_reg, i + j + D - 1, kb[(j + D - 1) % D], vb[(j + D - 1) % D],
                  ksr[(j + D - 1) % D], vsr[(j + D - 1) % D]);
        consume(BoolConst<false>{}, kb[j], vb[j], c0 + i + j, ksr[j], vsr[j]);
      }
    }
    // Fewer than 2D - 1 pages left; those before i + D - 1 are already loaded.
#pragma unroll
    for (int j = 0; j < 2 * D - 2; ++j) {
      if (i + j < n) {
        if (i + j + D - 1 < n)
          load_page(blk_reg, i + j + D - 1, kb[(j + D - 1) % D], vb[(j + D - 1) % D],
                    ksr[(j + D - 1) % D], vsr[(j + D - 1) % D]);
        if constexpr (ROPE) substitute_new_rows(kb[j % D], vb[j % D], c0 + i + j);
        consume(BoolConst<true>{}, kb[j % D], vb[j % D], c0 + i + j, ksr[j % D], vsr[j % D]);
      }
    }
  }

  // The staged rows to the pool, once this wave has read the page that holds their slot.
  if constexpr (ROPE) {
    if (staged) write_staged_rows<T, KV, DH, BS>(a, b, kvh, lane, new_k_s, new_v_s);
  }

  // Per-wave state: l summed over the 16 tokens, acc over the 4 token groups.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    l[i] = row16_sum(l[i]);
    const int h = grp * 4 + i;
    if (h < G && r == 0) {
      m_s[wave][h] = m[i];
      l_s[wave][h] = l[i];
    }
  }
#pragma unroll
  for (int j = 0; j < HPL; ++j)
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      acc[j][d] += __shfl_xor(acc[j][d], LPR, 64);
      acc[j][d] += __shfl_xor(acc[j][d], 2 * LPR, 64);
    }
  if (tg == 0) {
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
      float *dst = &acc_s[wave][hg * HPL + j][dc * 8];
      *reinterpret_cast<float4 *>(dst) = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
      *reinterpret_cast<float4 *>(dst + 4) =
          make_float4(acc[j][4], acc[j][5], acc[j][6], acc[j][7]);
    }
  }
  __syncthreads();

  // Merge the waves (a wave without pages has m = -inf, l = 0, acc = 0).
  const bool single = a.max_splits == 1;
  for (int i = threadIdx.x; i < G * DH; i += 64 * kWaves) {
    const int h = i / DH, d = i % DH;
    float M_ = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M_ = fmaxf(M_, m_s[w][h]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float e = m_s[w][h] == -INFINITY ? 0.f : fast_exp2(m_s[w][h] - M_);
      L += e * l_s[w][h];
      o += e * acc_s[w][h][d];
    }
    // v_scale (1 for pools in the model dtype, an exact no-op) decodes V.
    if (single) {
      out[b * a.o_ss + (int64_t)(kvh * G + h) * a.o_hs + d] = from_float<T>(o / L * a.v_scale);
    } else {
      const int64_t w = ((int64_t)b * a.num_q_heads + kvh * G + h) * a.max_splits + split;
      if (d == 0) {
        a.ws_m[w] = M_;
        a.ws_l[w] = L;
      }
      a.ws_acc[w * DH + d] = o * a.v_scale;
    }
  }
}

// ---------------------------------------------------------------------------
// P.V on the matrix cores, for pools in the model dtype (bf16 / fp16).
//
// Per page the score MFMA runs with its operands swapped: S (16 tokens x 16 head
// columns) = K . Q^T with v_mfma_f32_16x16x32 (A = the page's K rows, B = Q^T,
// column n being query head n % G), so lane (grp, r) holds the scores of tokens
// grp*4 .. +3 for head column r. After exp2 these are exactly the B operand of
// v_mfma_f32_16x16x16 for
//   O^T (16 dims x 16 head columns) += V^T (16 dims x 16 tokens) . P^T,
// one MFMA per 16 dims: P never goes through LDS, and the P.V dot products leave
// the VALU. K and V pages go HBM -> LDS with global_load_lds (a two-page ring per
// wave, the 16-byte chunks of each row XOR-swizzled as in the prefill kernel, so
// that neither operand read has bank conflicts) and come back as MFMA operands:
// K rows through ds_read_b128, V^T through ds_read_b64_tr_b16 (within each 16-lane
// group, lane j receives dim j of tokens 4g .. 4g+3 when lane 4e + q addresses dims
// 4q .. 4q+3 of token 4g + e). Every LDS read, and every wait for the page loads,
// is explicit inline asm: the compiler cannot tell ring slots apart and would wait
// for all loads in flight. A head column's softmax state is the same in the four
// lanes that hold it (the page maximum across the lane groups takes two lane
// swaps), so rescaling its accumulators stays in the lane.
// Pages per wave in the ring: the one consumed and those in flight behind it.
template <int DH, typename KV>
constexpr int D_of() {
  return DH == 64 ? 3 : 2;
}

// e4m3 K rows in LDS: 8-byte reads of 16 rows at one column would share banks, so
// the 16-byte chunks of row r are XOR-swizzled by r / 2 (Dh 128: 128-byte rows) or
// r / 4 (Dh 64: 64-byte rows). e4m3 V pages stay in load order: they are read back
// 16 bytes per lane, contiguously, to be decoded.
template <int DH>
__device__ __forceinline__ int pv_k8_swizzle(int row) {
  return DH == 128 ? ((row >> 1) & 7) : ((row >> 2) & 3);
}

// 16 e4m3 codes (four words) decoded exactly to T, as two 16-byte chunks of T.
template <typename T>
__device__ __forceinline__ void decode_fp8_chunk(u32x4 w, u32x4 &lo, u32x4 &hi) {
  uint32_t o[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const auto p0 = Dot2<T>::template from_fp8<false>(w[k]);
    const auto p1 = Dot2<T>::template from_fp8<true>(w[k]);
    __builtin_memcpy(&o[2 * k], &p0, 4);
    __builtin_memcpy(&o[2 * k + 1], &p1, 4);
  }
  lo = u32x4{o[0], o[1], o[2], o[3]};
  hi = u32x4{o[4], o[5], o[6], o[7]};
}
// Every page is read once: non-temporal loads.
constexpr int kPvLoadPolicy = kLdsNonTemporal;

template <int DH>
struct PvSwizzle {
  static __device__ __forceinline__ int k(int row) {
    return DH == 128 ? (row & 15) : ((row >> 1) & 7);
  }
  static __device__ __forceinline__ int v(int row) {
    return DH == 128 ? 2 * (row & 7) : (row & 7);
  }
};

#define TKS_S(x) #x
#define TKS_RD128(o, a, off) "ds_read_b128 %" TKS_S(o) ", %" TKS_S(a) " offset:%" TKS_S(off) "\n\t"
#define TKS_RDTR(o, a, off) "ds_read_b64_tr_b16 %" TKS_S(o) ", %" TKS_S(a) " offset:%" TKS_S(off) "\n\t"

// A page's operands from LDS ring offset OFF (bytes), after waiting until at most
// VM vector-memory operations of the wave are in flight (the page's loads are then
// done): keys() the K rows (one 16-byte read per 32 dims), values() the V^T
// operands (one 8-byte transposed read per 16 dims). The results are valid after
// wait(). (Compiled for the device only.)
template <int DH>
struct PvReads;
template <>
struct PvReads<128> {
  template <int VM, int OFF>
  static __device__ __forceinline__ void keys(const uint32_t (&ka)[4], u32x4 (&k)[4]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt vmcnt(%8)\n\t"
                 TKS_RD128(0, 4, 9) TKS_RD128(1, 5, 9) TKS_RD128(2, 6, 9) TKS_RD128(3, 7, 9)
                 : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3])
                 : "v"(ka[0]), "v"(ka[1]), "v"(ka[2]), "v"(ka[3]), "n"(VM), "i"(OFF)
                 : "memory");
#else
    (void)ka, (void)k;
#endif
  }
  template <int VM, int OFF>
  static __device__ __forceinline__ void values(const uint32_t (&va)[8], u32x2 (&v)[8]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt vmcnt(%16)\n\t"
                 TKS_RDTR(0, 8, 17) TKS_RDTR(1, 9, 17) TKS_RDTR(2, 10, 17) TKS_RDTR(3, 11, 17)
                 TKS_RDTR(4, 12, 17) TKS_RDTR(5, 13, 17) TKS_RDTR(6, 14, 17) TKS_RDTR(7, 15, 17)
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
                   "=&v"(v[6]), "=&v"(v[7])
                 : "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]), "v"(va[4]), "v"(va[5]),
                   "v"(va[6]), "v"(va[7]), "n"(VM), "i"(OFF)
                 : "memory");
#else
    (void)va, (void)v;
#endif
  }
  static __device__ __forceinline__ void wait(u32x4 (&k)[4]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(k[0]), "+v"(k[1]), "+v"(k[2]), "+v"(k[3])::"memory");
#else
    (void)k;
#endif
  }
  // The keys, with the page's 8 V^T reads issued behind them still in flight.
  static __device__ __forceinline__ void wait_before_values(u32x4 (&k)[4]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(k[0]), "+v"(k[1]), "+v"(k[2]), "+v"(k[3])::"memory");
#else
    (void)k;
#endif
  }
  static __device__ __forceinline__ void wait(u32x2 (&v)[8]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                   "+v"(v[6]), "+v"(v[7])::"memory");
#else
    (void)v;
#endif
  }
};
template <>
struct PvReads<64> {
  template <int VM, int OFF>
  static __device__ __forceinline__ void keys(const uint32_t (&ka)[2], u32x4 (&k)[2]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt vmcnt(%4)\n\t" TKS_RD128(0, 2, 5) TKS_RD128(1, 3, 5)
                 : "=&v"(k[0]), "=&v"(k[1])
                 : "v"(ka[0]), "v"(ka[1]), "n"(VM), "i"(OFF)
                 : "memory");
#else
    (void)ka, (void)k;
#endif
  }
  template <int VM, int OFF>
  static __device__ __forceinline__ void values(const uint32_t (&va)[4], u32x2 (&v)[4]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt vmcnt(%8)\n\t"
                 TKS_RDTR(0, 4, 9) TKS_RDTR(1, 5, 9) TKS_RDTR(2, 6, 9) TKS_RDTR(3, 7, 9)
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
                 : "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]), "n"(VM), "i"(OFF)
                 : "memory");
#else
    (void)va, (void)v;
#endif
  }
  static __device__ __forceinline__ void wait(u32x4 (&k)[2]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(k[0]), "+v"(k[1])::"memory");
#else
    (void)k;
#endif
  }
  static __device__ __forceinline__ void wait_before_values(u32x4 (&k)[2]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(k[0]), "+v"(k[1])::"memory");
#else
    (void)k;
#endif
  }
  static __device__ __forceinline__ void wait(u32x2 (&v)[4]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3])::"memory");
#else
    (void)v;
#endif
  }
};

// fp8 pools. kv_codes(): in one batch with one wait, the K rows as e4m3 codes (one
// 8-byte read per 32 dims) and the page's V codes, 16 bytes per lane per 1 KiB of
// page, in the order the HBM -> LDS loads wrote them (results valid on return);
// kv_codes_rows() adds the lane's four K and four V scales. staged_values():
// the codes decoded to T go to the wave's staging page (two 16-byte writes per 16
// codes, in the swizzled layout of pools in the model dtype), and the V^T operands are
// read back from it (valid after PvReads::wait); LDS operations of one wave complete
// in order, so the reads see the writes.
#define TKS_RD64(o, a, off) "ds_read_b64 %" TKS_S(o) ", %" TKS_S(a) " offset:%" TKS_S(off) "\n\t"
#define TKS_WR128(a, d) "ds_write_b128 %" TKS_S(a) ", %" TKS_S(d) "\n\t"
#define TKS_RDTR0(o, a) "ds_read_b64_tr_b16 %" TKS_S(o) ", %" TKS_S(a) "\n\t"
template <int DH>
struct PvReads8;
template <>
struct PvReads8<128> {
  // The page's K codes and its raw V codes in one batch (VM: the V tile's wait).
  template <int VM, int OFF, int VOFF>
  static __device__ __forceinline__ void kv_codes(const uint32_t (&ka)[4], u32x2 (&k)[4],
                                                  const uint32_t (&ra)[2], u32x4 (&v)[2]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt vmcnt(%12)\n\t"
                 "ds_read_b64 %0, %6 offset:%13\n\t"
                 "ds_read_b64 %1, %7 offset:%13\n\t"
                 "ds_read_b64 %2, %8 offset:%13\n\t"
                 "ds_read_b64 %3, %9 offset:%13\n\t"
                 "ds_read_b128 %4, %10 offset:%14\n\t"
                 "ds_read_b128 %5, %11 offset:%14\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(v[0]), "=&v"(v[1])
                 : "v"(ka[0]), "v"(ka[1]), "v"(ka[2]), "v"(ka[3]), "v"(ra[0]), "v"(ra[1]),
                   "n"(VM), "i"(OFF), "i"(VOFF)
                 : "memory");
#else
    (void)ka, (void)k, (void)ra, (void)v;
#endif
  }
  template <int VM, int OFF, int VOFF>
  static __device__ __forceinline__ void kv_codes_rows(const uint32_t (&ka)[4], u32x2 (&k)[4],
                                                       const uint32_t (&ra)[2], u32x4 (&v)[2],
                                                       uint32_t sa, u32x4 &ks, u32x4 &vs) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt vmcnt(%15)\n\t"
                 "ds_read_b64 %0, %8 offset:%16\n\t"
                 "ds_read_b64 %1, %9 offset:%16\n\t"
                 "ds_read_b64 %2, %10 offset:%16\n\t"
                 "ds_read_b64 %3, %11 offset:%16\n\t"
                 "ds_read_b128 %4, %12 offset:%18\n\t"
                 "ds_read_b128 %5, %13 offset:%18\n\t"
                 "ds_read_b128 %6, %14 offset:%16\n\t"
                 "ds_read_b128 %7, %14 offset:%17\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(v[0]), "=&v"(v[1]),
                   "=&v"(ks), "=&v"(vs)
                 : "v"(ka[0]), "v"(ka[1]), "v"(ka[2]), "v"(ka[3]), "v"(ra[0]), "v"(ra[1]),
                   "v"(sa), "n"(VM), "i"(OFF), "i"(OFF + 64), "i"(VOFF)
                 : "memory");
#else
    (void)ka, (void)k, (void)ra, (void)v, (void)sa, (void)ks, (void)vs;
#endif
  }
  static __device__ __forceinline__ void staged_values(const uint32_t (&wa)[4], const u32x4 (&d)[4],
                                                       const uint32_t (&va)[8], u32x2 (&v)[8]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile(TKS_WR128(8, 12) TKS_WR128(9, 13) TKS_WR128(10, 14) TKS_WR128(11, 15)
                 TKS_RDTR0(0, 16) TKS_RDTR0(1, 17) TKS_RDTR0(2, 18) TKS_RDTR0(3, 19)
                 TKS_RDTR0(4, 20) TKS_RDTR0(5, 21) TKS_RDTR0(6, 22) TKS_RDTR0(7, 23)
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
                   "=&v"(v[6]), "=&v"(v[7])
                 : "v"(wa[0]), "v"(wa[1]), "v"(wa[2]), "v"(wa[3]), "v"(d[0]), "v"(d[1]),
                   "v"(d[2]), "v"(d[3]), "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]),
                   "v"(va[4]), "v"(va[5]), "v"(va[6]), "v"(va[7])
                 : "memory");
#else
    (void)wa, (void)d, (void)va, (void)v;
#endif
  }
};
template <>
struct PvReads8<64> {
  template <int VM, int OFF, int VOFF>
  static __device__ __forceinline__ void kv_codes(const uint32_t (&ka)[2], u32x2 (&k)[2],
                                                  const uint32_t (&ra)[1], u32x4 (&v)[1]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt vmcnt(%6)\n\t"
                 "ds_read_b64 %0, %3 offset:%7\n\t"
                 "ds_read_b64 %1, %4 offset:%7\n\t"
                 "ds_read_b128 %2, %5 offset:%8\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(k[0]), "=&v"(k[1]), "=&v"(v[0])
                 : "v"(ka[0]), "v"(ka[1]), "v"(ra[0]), "n"(VM), "i"(OFF), "i"(VOFF)
                 : "memory");
#else
    (void)ka, (void)k, (void)ra, (void)v;
#endif
  }
  template <int VM, int OFF, int VOFF>
  static __device__ __forceinline__ void kv_codes_rows(const uint32_t (&ka)[2], u32x2 (&k)[2],
                                                       const uint32_t (&ra)[1], u32x4 (&v)[1],
                                                       uint32_t sa, u32x4 &ks, u32x4 &vs) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt vmcnt(%9)\n\t"
                 "ds_read_b64 %0, %5 offset:%10\n\t"
                 "ds_read_b64 %1, %6 offset:%10\n\t"
                 "ds_read_b128 %2, %7 offset:%12\n\t"
                 "ds_read_b128 %3, %8 offset:%10\n\t"
                 "ds_read_b128 %4, %8 offset:%11\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(k[0]), "=&v"(k[1]), "=&v"(v[0]), "=&v"(ks), "=&v"(vs)
                 : "v"(ka[0]), "v"(ka[1]), "v"(ra[0]), "v"(sa), "n"(VM), "i"(OFF), "i"(OFF + 64),
                   "i"(VOFF)
                 : "memory");
#else
    (void)ka, (void)k, (void)ra, (void)v, (void)sa, (void)ks, (void)vs;
#endif
  }
  static __device__ __forceinline__ void staged_values(const uint32_t (&wa)[2], const u32x4 (&d)[2],
                                                       const uint32_t (&va)[4], u32x2 (&v)[4]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile(TKS_WR128(4, 6) TKS_WR128(5, 7)
                 TKS_RDTR0(0, 8) TKS_RDTR0(1, 9) TKS_RDTR0(2, 10) TKS_RDTR0(3, 11)
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
                 : "v"(wa[0]), "v"(wa[1]), "v"(d[0]), "v"(d[1]), "v"(va[0]), "v"(va[1]),
                   "v"(va[2]), "v"(va[3])
                 : "memory");
#else
    (void)wa, (void)d, (void)va, (void)v;
#endif
  }
};
#undef TKS_RD64
#undef TKS_WR128
#undef TKS_RDTR0

#undef TKS_RD128
#undef TKS_RDTR
#undef TKS_S

// LDS reads that complete before the statement ends, for the fused append's staged
// rows (asm, so they stay inside the branch that needs them instead of being
// hoisted where the compiler would make them wait for the page loads in flight).
__device__ __forceinline__ uint4 lds_read16_now(const void *p) {
  u32x4 v = {0u, 0u, 0u, 0u};
#if __HIP_DEVICE_COMPILE__
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_address(p)) : "memory");
#else
  (void)p;
#endif
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t lds_read2_now(const void *p) {
  uint32_t v = 0u;
#if __HIP_DEVICE_COMPILE__
  asm volatile("ds_read_u16 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_address(p)) : "memory");
#else
  (void)p;
#endif
  return v;
}

__device__ __forceinline__ uint32_t lds_read1_now(const void *p) {
  uint32_t v = 0u;
#if __HIP_DEVICE_COMPILE__
  asm volatile("ds_read_u8 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_address(p)) : "memory");
#else
  (void)p;
#endif
  return v;
}
__device__ __forceinline__ uint2 lds_read8_now(const void *p) {
  u32x2 v = {0u, 0u};
#if __HIP_DEVICE_COMPILE__
  asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_address(p)) : "memory");
#else
  (void)p;
#endif
  return make_uint2(v[0], v[1]);
}

template <int N>
struct IntConst {
  static constexpr int value = N;
};

// Waves per SIMD the register budget is cut for. At Dh 64 LDS holds three
// workgroups per CU, and asking for three waves keeps the P.V accumulators in
// VGPRs (left to itself the compiler put them in AGPRs, with a copy per access:
// fp8 serving shape 10.4 -> 10.0 us). At Dh 128 the budget is left alone: three
// waves per SIMD over fp8 pools (145 VGPRs) ran the Llama-3-8B decode batch 3 %
// slower (152.5 vs 148.7 us).
template <int DH>
constexpr int kPvMinWaves = DH == 64 ? 3 : 1;

// ROWS: fp8 pools with one scale per pool row (a.k_rs, a.v_rs): a page's 16 K and 16
// V scales ride in the ring with it; a lane multiplies its scores by its tokens' K
// scales and its probabilities, after they enter the row sum, by their V scales.
template <typename T, typename KV, int DH, int G, bool ROPE, bool ROWS = false>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(kPvMinWaves<DH>)))
void decode_pv_kernel(DecodeArgs a) {
  constexpr bool kFp8 = sizeof(KV) == 1;
  static_assert(!ROWS || kFp8, "row scales: fp8 pools");
  constexpr int BS = 16, NC = DH / 32, DT = DH / 16, CPR = DH / 8;
  constexpr int kPage = BS * DH;                        // elements of one K (or V) page
  constexpr int kRowBytes = DH * (int)sizeof(KV);       // one pool row as stored
  constexpr int CPRR = kRowBytes / 16;                  // its 16-byte chunks
  constexpr int kPageBytes = BS * kRowBytes;
  // ROWS: one 4-byte load per lane of the page's 16 K and 16 V scales (lanes 32-63
  // repeat lanes 0-31), so the K scales sit at the area's start and the V scales 64
  // bytes on.
  constexpr int kScaleBytes = ROWS ? 4 * 64 : 0;
  constexpr int kStageBytes = 2 * kPageBytes + kScaleBytes;  // K page, V page, scales
  constexpr int L = kPageBytes / (16 * 64);             // HBM -> LDS loads per page tile
  // A page's loads, in issue order: its scales (ROWS), its K tile, its V tile.
  constexpr int kTileOps = L;
  constexpr int kPageOps = 2 * L + (ROWS ? 1 : 0);
  // fp8 pools: each wave decodes its current V page into a staging page of T, laid
  // out as a page of a pool in the model dtype (the V^T reads are the same).
  constexpr int kStagingBytes = kFp8 ? kPage * (int)sizeof(T) : 0;
  constexpr int kWaveBytes = D_of<DH, KV>() * kStageBytes + kStagingBytes;
  constexpr int D = D_of<DH, KV>();
  static_assert(D == 2 || D == 3, "ring depth");
  static_assert(16 % G == 0 && (DH == 64 || DH == 128) && L >= 1, "shape");
  using M = Mfma<T>;
  using IO = PageIO<T, KV>;
  using Swz = PvSwizzle<DH>;
  using Reads = PvReads<DH>;
  using Reads8 = PvReads8<DH>;
  typedef typename M::f4 f4;
  typedef typename M::v4 v4;
  // The ring, reused after the page loop for the waves' partial results.
  constexpr int kRingBytes = kWaves * kWaveBytes;
  constexpr int kMergeBytes = kWaves * G * (DH + 2) * (int)sizeof(float);
  static_assert(kMergeBytes <= kRingBytes, "merge area");
  __shared__ __attribute__((aligned(16))) char ring[kRingBytes];
  __shared__ __attribute__((aligned(16))) KV new_k_s[ROPE ? DH : 1];
  __shared__ __attribute__((aligned(16))) KV new_v_s[ROPE ? DH : 1];
  __shared__ float new_scale_s[(ROPE && ROWS) ? 2 : 1];  // the staged rows' K, V scales
  __shared__ __attribute__((aligned(16))) T q_s[G * DH];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;    // K rows: token r; S and O^T: head column r
  const int grp = lane >> 4;  // K: dims grp*8 of each 32; S: tokens grp*4 .. +3; O^T: dims

  // Work item (rank, KV head) of this workgroup. ROWS with an even KV-head count: the
  // 16 K (or V) scales of a page are 64 bytes, and the two KV heads of one 128-byte
  // line go to workgroups 8 apart, i.e. dispatched one after the other on the same
  // XCD (workgroup i runs on XCD i % 8), so the line comes from HBM once for both. A
  // bijection on each whole 16 items of a split; the rest keep their places.
  int kvh_i = blockIdx.x, rank_i = blockIdx.y;
  if constexpr (ROWS) {
    const int X = gridDim.x;
    const int l = blockIdx.x + X * (int)blockIdx.y;
    if ((X & 1) == 0 && l < ((X * (int)gridDim.y) & ~15)) {
      const int item = 2 * ((l >> 4) * 8 + (l & 7)) + ((l >> 3) & 1);
      kvh_i = item % X;
      rank_i = item / X;
    }
  }
  const int kvh = kvh_i;
  const int split = blockIdx.z;
  const int b = a.seq_order ? min(max(a.seq_order[rank_i], 0), (int)gridDim.y - 1) : rank_i;
  // A length above the host bound is clamped so no access can leave its buffer.
  const int len = min(a.seq_lens[b], a.key_cap);
  const int n_pages = (len + BS - 1) / BS;
  const int p_begin = split * a.pages_per_split;
  T *out = static_cast<T *>(a.out);
  if (p_begin >= n_pages) {
    if (split == 0) {  // empty sequence: defined all-zero output
      for (int i = threadIdx.x; i < G * DH; i += 64 * kWaves)
        out[b * a.o_ss + (int64_t)(kvh * G + i / DH) * a.o_hs + i % DH] = from_float<T>(0.f);
      if constexpr (ROPE) {
        if (n_pages == 0 && threadIdx.x < 64 &&
            stage_new_rows<T, KV, DH, BS, ROWS>(a, b, kvh, threadIdx.x, new_k_s, new_v_s,
                                                new_scale_s)) {
          wave_lds_sync();
          write_staged_rows<T, KV, DH, BS, ROWS>(a, b, kvh, threadIdx.x, new_k_s, new_v_s,
                                                 new_scale_s);
        }
      }
    }
    return;
  }
  const int p_end = min(n_pages, p_begin + a.pages_per_split);
  const int per_wave = (p_end - p_begin + kWaves - 1) / kWaves;
  const int w_begin = p_begin + wave * per_wave;
  const int w_end = min(p_end, w_begin + per_wave);

  // Q^T operands through LDS as in decode_mfma_kernel (rotated there when the RoPE
  // is fused in; the wave holding the sequence's last page stages the new rows).
  typename M::v8 qa[NC];
  const int32_t *bt_row = a.bt + (int64_t)b * a.bt_stride;
  bool staged = false;
  bool patch = false;
  const int new_off = ROPE ? (len - 1) % BS : 0;
  float new_ks = 1.f, new_vs = 1.f;  // ROWS: the staged rows' scales, in registers
  {
    const int t = threadIdx.x;
    if constexpr (ROPE) {
      constexpr int HALF = DH / 2;
      if (w_begin < w_end && w_end == n_pages) {  // wave-uniform
        staged = stage_new_rows<T, KV, DH, BS, ROWS>(a, b, kvh, lane, new_k_s, new_v_s,
                                                     new_scale_s);
        patch = staged && a.seq_lens[b] == len;
        wave_lds_sync();
        if constexpr (ROWS) {
          if (staged) {
            new_ks = new_scale_s[0];
            new_vs = new_scale_s[1];
          }
        }
      }
      if (t < G * HALF / 8) {
        const int64_t pos = min(max(a.positions[b], (int64_t)0), a.table_len - 1);
        const int h = t / (HALF / 8), j = (t % (HALF / 8)) * 8;
        const T *qrow =
            static_cast<const T *>(a.q) + b * a.q_ss + (int64_t)(kvh * G + h) * a.q_hs;
        float cf[8], sf[8], o1[8], o2[8];
        load_table<T, 8>(static_cast<const T *>(a.cos_t) + pos * HALF,
                         static_cast<const T *>(a.sin_t) + pos * HALF, j, cf, sf);
        rotate_values<T, 8>(qrow + j, cf, sf, HALF, o1, o2);
        st16(&q_s[h * DH + j], pack<T>(o1));
        st16(&q_s[h * DH + j + HALF], pack<T>(o2));
      }
    } else {
      if (t < G * DH / 8) {
        const int h = t / (DH / 8), j = (t % (DH / 8)) * 8;
        const T *qrow =
            static_cast<const T *>(a.q) + b * a.q_ss + (int64_t)(kvh * G + h) * a.q_hs;
        st16(&q_s[h * DH + j], ld16(qrow + j));
      }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NC; ++c) qa[c] = as_v8<T>(ld16(&q_s[(r % G) * DH + c * 32 + grp * 8]));
  }

  const char *kcb = reinterpret_cast<const char *>(static_cast<const KV *>(a.kc) + a.pool.layer_base +
                                                   (int64_t)kvh * a.pool.head_stride);
  const char *vcb = reinterpret_cast<const char *>(static_cast<const KV *>(a.vc) + a.pool.layer_base +
                                                   (int64_t)kvh * a.pool.head_stride);
  const int64_t block_bytes = a.pool.block_stride * (int64_t)sizeof(KV);
  // ROWS: the scales of token 0 of this head's page in block 0; a block's are
  // rows_per_block floats further.
  const int64_t rows_per_block = a.pool.block_stride / DH;
  const float *ks_page = nullptr;
  const float *vs_page = nullptr;
  if constexpr (ROWS) {
    const int64_t base = (a.pool.layer_base + (int64_t)kvh * a.pool.head_stride) / DH;
    ks_page = a.k_rs + base;
    vs_page = a.v_rs + base;
  }
  auto k_swizzle = [](int row) { return kFp8 ? pv_k8_swizzle<DH>(row) : Swz::k(row); };
  // Load j of a page tile fills 16-byte LDS slot j*64 + lane = row * CPRR + physical
  // chunk, with logical chunk physical ^ swizzle(row) of that row.
  uint32_t k_src[L], v_src[L];
#pragma unroll
  for (int j = 0; j < L; ++j) {
    const int slot = j * 64 + lane;
    const int row = slot / CPRR;
    k_src[j] = row * kRowBytes + ((slot % CPRR) ^ k_swizzle(row)) * 16;
    v_src[j] = row * kRowBytes + ((slot % CPRR) ^ (kFp8 ? 0 : Swz::v(row))) * 16;
  }
  // Operand addresses in ring slot 0 of this wave (the other slots and the V page are
  // immediate offsets). K: lane (grp, r) reads token r, dims c*32 + grp*8 .. +8.
  // V^T: lane (grp, r) addresses token grp*4 + r/4, dims t*16 + 4 (r % 4) .. +3, in the
  // V page (pools in the model dtype) or in the staging page (fp8 pools).
  char *wring = ring + wave * kWaveBytes;
  const uint32_t ring0 = lds_address(wring);
  const uint32_t stage0 = ring0 + D * kStageBytes;
  // ROWS: this lane's K scales in ring slot 0 (the V scales 64 bytes on).
  const uint32_t scale_addr = ring0 + 2 * kPageBytes + grp * 16;
  uint32_t ka[NC], va[DT];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if constexpr (kFp8)
      ka[c] = ring0 + r * kRowBytes + (((2 * c + grp / 2) ^ k_swizzle(r)) * 16) + (grp & 1) * 8;
    else
      ka[c] = ring0 + (r * CPR + ((c * 4 + grp) ^ Swz::k(r))) * 16;
  }
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    const int row = grp * 4 + r / 4;
    const int lc = t * 2 + (r % 4) / 2;
    va[t] = (kFp8 ? stage0 : ring0) + (row * CPR + (lc ^ Swz::v(row))) * 16 + (r & 1) * 8;
  }
  // fp8 pools: lane's 16-byte chunks j*64 + lane of the V page (16 codes of one row)
  // and where their decoded values go in the staging page.
  uint32_t vra[L], vwa[2 * L];
#pragma unroll
  for (int j = 0; j < L; ++j) {
    const int slot = j * 64 + lane;
    const int row = slot / CPRR, k = slot % CPRR;
    vra[j] = ring0 + slot * 16;
    vwa[2 * j] = stage0 + (row * CPR + ((2 * k) ^ Swz::v(row))) * 16;
    vwa[2 * j + 1] = stage0 + (row * CPR + ((2 * k + 1) ^ Swz::v(row))) * 16;
  }

  f4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  // Softmax state of head column r (equal in the column's four lanes): m = the
  // reference max in log2 units (-inf before the first key), thr = m + 8 (a score
  // above it moves the reference), mref = the value subtracted before exp2 (m, or
  // 0 while m is -inf), l = this lane's share of the sum (its tokens of each page).
  float m = -INFINITY, l = 0.f, thr = -INFINITY, mref = 0.f;
  const float scale_log2 = a.scale_log2;

  // Page idx of the chunk's block-id register into ring slot SLOT: its K tile, then
  // its V tile (2 L loads, in that order).
  auto issue = [&](auto slot_c, int blk_reg, int idx) {
    constexpr int SLOT = decltype(slot_c)::value;
    const int64_t blk = clamp_block(__builtin_amdgcn_readlane(blk_reg, idx), a.pool.num_blocks);
    const char *kp = kcb + blk * block_bytes;
    const char *vp = vcb + blk * block_bytes;
    if constexpr (ROWS) {
      const float *src = ((lane & 31) < 16 ? ks_page : vs_page) + blk * rows_per_block + (lane & 15);
      load_lds4<kPvLoadPolicy>(src, wring + SLOT * kStageBytes + 2 * kPageBytes);
    }
#pragma unroll
    for (int j = 0; j < L; ++j)
      load_lds16<kPvLoadPolicy>(kp + k_src[j], wring + SLOT * kStageBytes + j * 1024);
#pragma unroll
    for (int j = 0; j < L; ++j)
      load_lds16<kPvLoadPolicy>(vp + v_src[j], wring + SLOT * kStageBytes + kPageBytes + j * 1024);
  };
  // after: pages whose loads (2 L each) were issued after this page's (0 .. D-1).
  auto consume = [&](auto check_end, auto slot_c, int p, int after) {
    constexpr bool kCheckEnd = decltype(check_end)::value;
    constexpr int SLOT = decltype(slot_c)::value;
    constexpr int KOFF = SLOT * kStageBytes, VOFF = KOFF + kPageBytes;
    f4 s4 = {0.f, 0.f, 0.f, 0.f};
    float ks4[4] = {1.f, 1.f, 1.f, 1.f}, vs4[4] = {1.f, 1.f, 1.f, 1.f};
    u32x4 raw[kFp8 ? L : 1];  // fp8 pools: the page's V codes, read with its K codes
    // The page's V^T operands (pools in the model dtype: requested with its K rows).
    u32x2 vt[DT];
    if constexpr (kFp8) {
      u32x2 kr[NC];
      if constexpr (ROWS) {
        // This lane's tokens' K and V scales, read with the K codes (their load was
        // issued before the K tile's, so the same wait covers it).
        u32x4 ku, vu;
        if (D > 2 && after >= 2)
          Reads8::template kv_codes_rows<2 * kPageOps, KOFF, VOFF>(ka, kr, vra, raw, scale_addr, ku, vu);
        else if (after >= 1)
          Reads8::template kv_codes_rows<kPageOps, KOFF, VOFF>(ka, kr, vra, raw, scale_addr, ku, vu);
        else
          Reads8::template kv_codes_rows<0, KOFF, VOFF>(ka, kr, vra, raw, scale_addr, ku, vu);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ks4[i] = __uint_as_float(ku[i]);
          vs4[i] = __uint_as_float(vu[i]);
        }
        if constexpr (ROPE) {  // the new token's scales in place of its slot's
          if (patch && p == n_pages - 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              ks4[i] = grp * 4 + i == new_off ? new_ks : ks4[i];
              vs4[i] = grp * 4 + i == new_off ? new_vs : vs4[i];
            }
          }
        }
      } else {
        if (D > 2 && after >= 2)
          Reads8::template kv_codes<2 * kPageOps, KOFF, VOFF>(ka, kr, vra, raw);
        else if (after >= 1)
          Reads8::template kv_codes<kPageOps, KOFF, VOFF>(ka, kr, vra, raw);
        else
          Reads8::template kv_codes<0, KOFF, VOFF>(ka, kr, vra, raw);
      }
      if constexpr (ROPE) {
        // The new token's K codes in place of what was loaded of its slot.
        if (patch && p == n_pages - 1 && r == new_off) {
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const uint2 u = lds_read8_now(new_k_s + c * 32 + grp * 8);
            kr[c] = u32x2{u.x, u.y};
          }
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c)
        s4 = M::run(IO::k_operand(make_uint2(kr[c][0], kr[c][1])), qa[c], s4);
    } else {
      u32x4 kr[NC];
      if (D > 2 && after >= 2) {
        Reads::template keys<kTileOps + 2 * kPageOps, KOFF>(ka, kr);
        Reads::template values<2 * kPageOps, VOFF>(va, vt);
      } else if (after >= 1) {
        Reads::template keys<kTileOps + kPageOps, KOFF>(ka, kr);
        Reads::template values<kPageOps, VOFF>(va, vt);
      } else {
        Reads::template keys<kTileOps, KOFF>(ka, kr);
        Reads::template values<0, VOFF>(va, vt);
      }
      Reads::wait_before_values(kr);
      if constexpr (ROPE) {
        // The new token's K row in place of what was loaded of its slot.
        if (patch && p == n_pages - 1 && r == new_off) {
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const uint4 u = lds_read16_now(new_k_s + c * 32 + grp * 8);
            kr[c] = u32x4{u.x, u.y, u.z, u.w};
          }
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c)
        s4 = M::run(as_v8<T>(make_uint4(kr[c][0], kr[c][1], kr[c][2], kr[c][3])), qa[c], s4);
    }
    // fp8 pools: the page's V codes are decoded into the staging page, and the V^T
    // operands read back from it, used after the softmax.
    if constexpr (kFp8) {
      u32x4 dec[2 * L];
#pragma unroll
      for (int j = 0; j < L; ++j) decode_fp8_chunk<T>(raw[j], dec[2 * j], dec[2 * j + 1]);
      Reads8::staged_values(vwa, dec, va, vt);
    }
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = s4[i] * scale_log2;
    if constexpr (ROWS) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] *= ks4[i];
    }
    // The sequence's last page (uniform): keys past len score -inf, and their V
    // values, whatever the pool holds there, become 0 below (0 * NaN is NaN).
    const bool tail = kCheckEnd && (p + 1) * BS > len;
    if (tail) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool valid = p * BS + grp * 4 + i < len;
        sv[i] = valid ? sv[i] : -INFINITY;
        if constexpr (ROWS) vs4[i] = valid ? vs4[i] : 0.f;  // an unwritten row's scale may be NaN
      }
    }
    bool over = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) over = over || sv[i] > thr;
    // A score more than 8 above its column's reference (every column on the first
    // page): page maxima, new references, l and the accumulators rescaled.
    if (__builtin_amdgcn_ballot_w64(over) != 0) {
      const float mx = xgroup_max(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
      const bool bump = mx > thr;
      const float alpha = bump ? fast_exp2(m - mx) : 1.f;
      m = bump ? mx : m;
      thr = m + 8.f;
      mref = m == -INFINITY ? 0.f : m;
      l *= alpha;
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] *= alpha;
    }
    float pv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pv[i] = fast_exp2(sv[i] - mref);
    l += (pv[0] + pv[1]) + (pv[2] + pv[3]);
    v4 pb;
#pragma unroll
    for (int i = 0; i < 4; ++i) pb[i] = static_cast<typename M::elem>(ROWS ? pv[i] * vs4[i] : pv[i]);
    Reads::wait(vt);
    if (tail) {
      const int base = p * BS + grp * 4;
      const uint32_t keep_lo = (base < len ? 0x0000FFFFu : 0u) | (base + 1 < len ? 0xFFFF0000u : 0u);
      const uint32_t keep_hi = (base + 2 < len ? 0x0000FFFFu : 0u) | (base + 3 < len ? 0xFFFF0000u : 0u);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        vt[t][0] &= keep_lo;
        vt[t][1] &= keep_hi;
      }
    }
    if constexpr (ROPE) {
      // The new token's V row: element e of lane (grp, r) is token grp*4 + e.
      const int e = new_off - grp * 4;
      if (patch && p == n_pages - 1 && e >= 0 && e < 4) {
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          uint32_t nv;
          if constexpr (kFp8) {
            const auto pr = Dot2<T>::template from_fp8<false>(lds_read1_now(new_v_s + t * 16 + r));
            uint32_t both;
            __builtin_memcpy(&both, &pr, 4);
            nv = both & 0xFFFFu;
          } else {
            nv = lds_read2_now(new_v_s + t * 16 + r);
          }
          const int w = e >> 1, sh = (e & 1) * 16;
          vt[t][w] = (vt[t][w] & ~(0xFFFFu << sh)) | (nv << sh);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      v4 vop;
      __builtin_memcpy(&vop, &vt[t], 8);
      acc[t] = M::run16(vop, pb, acc[t]);
    }
  };

  for (int c0 = w_begin; c0 < w_end; c0 += 64) {
    const int n = min(w_end, c0 + 64) - c0;
    const int blk_reg = lane < n ? bt_row[c0 + lane] : 0;
    // The block ids, and everything else, before any page load is in flight: the
    // waits below count only page loads.
    __builtin_amdgcn_s_waitcnt(0);
    issue(IntConst<0>{}, blk_reg, 0);
    if (D > 2 && n > 1) issue(IntConst<1 % D>{}, blk_reg, 1);
    int i = 0;  // page i sits in ring slot i % D
    // Steady state: D pages per iteration, each consumed with the next D - 1 in flight.
    for (; i + 2 * D - 1 <= n; i += D) {
      issue(IntConst<(D - 1) % D>{}, blk_reg, i + D - 1);
      consume(BoolConst<false>{}, IntConst<0>{}, c0 + i, D - 1);
      issue(IntConst<D % D>{}, blk_reg, i + D);
      consume(BoolConst<false>{}, IntConst<1 % D>{}, c0 + i + 1, D - 1);
      if constexpr (D > 2) {
        issue(IntConst<(D + 1) % D>{}, blk_reg, i + D + 1);
        consume(BoolConst<false>{}, IntConst<2 % D>{}, c0 + i + 2, D - 1);
      }
    }
    // Fewer than 2 D - 1 pages left; those before i + D - 1 are in flight.
    auto drain = [&](auto j_c) {
      constexpr int j = decltype(j_c)::value;
      if (i + j < n) {
        if (i + j + D - 1 < n) issue(IntConst<(j + D - 1) % D>{}, blk_reg, i + j + D - 1);
        consume(BoolConst<true>{}, IntConst<j % D>{}, c0 + i + j, min(D - 1, n - 1 - (i + j)));
      }
    };
    drain(IntConst<0>{});
    drain(IntConst<1>{});
    if constexpr (D > 2) {
      drain(IntConst<2>{});
      drain(IntConst<3>{});
    }
  }

  // The staged rows to the pool, once this wave has read the page that holds their slot.
  if constexpr (ROPE) {
    if (staged)
      write_staged_rows<T, KV, DH, BS, ROWS>(a, b, kvh, lane, new_k_s, new_v_s, new_scale_s);
  }

  // Per-wave state, in the ring's memory once every wave is done with it: l summed
  // over the four lane groups; lanes of columns r < G hold head r's dims
  // t*16 + grp*4 .. +3.
  l = xgroup_sum(l);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  float *m_s = reinterpret_cast<float *>(ring);        // [kWaves][G]
  float *l_s = m_s + kWaves * G;                        // [kWaves][G]
  float *acc_s = l_s + kWaves * G;                      // [kWaves][G][DH]
  if (r < G) {
    if (grp == 0) {
      m_s[wave * G + r] = m;
      l_s[wave * G + r] = l;
    }
#pragma unroll
    for (int t = 0; t < DT; ++t)
      *reinterpret_cast<float4 *>(&acc_s[(wave * G + r) * DH + t * 16 + grp * 4]) =
          make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
  }
  __syncthreads();

  // Merge the waves (a wave without pages has m = -inf, l = 0, acc = 0).
  const bool single = a.max_splits == 1;
  for (int i = threadIdx.x; i < G * DH; i += 64 * kWaves) {
    const int h = i / DH, d = i % DH;
    float M_ = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M_ = fmaxf(M_, m_s[w * G + h]);
    float L_ = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float e = m_s[w * G + h] == -INFINITY ? 0.f : fast_exp2(m_s[w * G + h] - M_);
      L_ += e * l_s[w * G + h];
      o += e * acc_s[(w * G + h) * DH + d];
    }
    // v_scale (1 for pools in the model dtype, an exact no-op) decodes V.
    if (single) {
      out[b * a.o_ss + (int64_t)(kvh * G + h) * a.o_hs + d] = from_float<T>(o / L_ * a.v_scale);
    } else {
      const int64_t w = ((int64_t)b * a.num_q_heads + kvh * G + h) * a.max_splits + split;
      if (d == 0) {
        a.ws_m[w] = M_;
        a.ws_l[w] = L_;
      }
      a.ws_acc[w * DH + d] = o * a.v_scale;
    }
  }
}

// Pools in the model dtype take the P.V-on-MFMA kernel.
constexpr bool kPvMfma = true;

template <typename T, typename KV, bool ROPE = false>
int32_t launch_typed(const DecodeArgs &a, int32_t num_seqs, int32_t num_kv_heads, int32_t G,
                     int32_t head_dim, hipStream_t s) {
  // KV heads vary fastest (consecutive workgroups, dealt round-robin over the
  // XCDs, carry equal work), splits slowest.
  const dim3 grid(num_kv_heads, num_seqs, a.max_splits);
#define TKS_DECODE(DH, GG)                                                          \
  if (head_dim == DH && G == GG) {                                                  \
    if constexpr (sizeof(KV) == 1) {                                                \
      if (a.k_rs != nullptr) {                                                      \
        if constexpr (kPvMfma || ROPE)                                              \
          decode_pv_kernel<T, KV, DH, GG, ROPE, true><<<grid, 64 * kWaves, 0, s>>>(a); \
        else                                                                        \
          decode_mfma_kernel<T, KV, DH, GG, false, true><<<grid, 64 * kWaves, 0, s>>>(a); \
        return check_launch();                                                      \
      }                                                                             \
    }                                                                               \
    if constexpr (kPvMfma) {                                                        \
      decode_pv_kernel<T, KV, DH, GG, ROPE><<<grid, 64 * kWaves, 0, s>>>(a);        \
    } else {                                                                        \
      decode_mfma_kernel<T, KV, DH, GG, ROPE><<<grid, 64 * kWaves, 0, s>>>(a);      \
    }                                                                               \
    return check_launch();                                                          \
  }
  TKS_DECODE(128, 4)
  TKS_DECODE(128, 8)
  TKS_DECODE(128, 2)
  TKS_DECODE(128, 1)
  TKS_DECODE(64, 8)
  TKS_DECODE(64, 4)
  TKS_DECODE(64, 2)
  TKS_DECODE(64, 16)
#undef TKS_DECODE
  return TKS_ERR_VALUE;
}

}  // namespace

bool decode_mfma_supported(int32_t dtype, int32_t head_dim, int32_t group) {
  if (dtype != TKS_BFLOAT16 && dtype != TKS_FLOAT16) return false;
  if (head_dim == 128) return group == 1 || group == 2 || group == 4 || group == 8;
  if (head_dim == 64) return group == 2 || group == 4 || group == 8 || group == 16;
  return false;
}

int32_t launch_decode_mfma(const DecodeArgs &a, int32_t dtype, int32_t num_seqs,
                           int32_t num_kv_heads, int32_t group, int32_t head_dim,
                           hipStream_t stream, bool fp8_pools) {
  if (a.positions != nullptr && fp8_pools)
    return dtype == TKS_BFLOAT16
               ? launch_typed<bf16_t, fp8e4m3_t, true>(a, num_seqs, num_kv_heads, group,
                                                       head_dim, stream)
               : launch_typed<_Float16, fp8e4m3_t, true>(a, num_seqs, num_kv_heads, group,
                                                         head_dim, stream);
  if (a.positions != nullptr) {
    return dtype == TKS_BFLOAT16
               ? launch_typed<bf16_t, bf16_t, true>(a, num_seqs, num_kv_heads, group, head_dim,
                                                    stream)
               : launch_typed<_Float16, _Float16, true>(a, num_seqs, num_kv_heads, group,
                                                        head_dim, stream);
  }
  if (fp8_pools)
    return dtype == TKS_BFLOAT16
               ? launch_typed<bf16_t, fp8e4m3_t>(a, num_seqs, num_kv_heads, group, head_dim, stream)
               : launch_typed<_Float16, fp8e4m3_t>(a, num_seqs, num_kv_heads, group, head_dim,
                                                   stream);
  return dtype == TKS_BFLOAT16
             ? launch_typed<bf16_t, bf16_t>(a, num_seqs, num_kv_heads, group, head_dim, stream)
             : launch_typed<_Float16, _Float16>(a, num_seqs, num_kv_heads, group, head_dim,
                                                stream);
}

}  // namespace tks
